// zz_route.hip -- MoE front half on gfx950: input norms + int8 activation
// quantisation, router logits, certified top-k gating, and the batch-union
// dispatch (histogram / prefix / stable scatter as one LDS sort).
//
// Exactness strategy. The reference computes its routing decisions with serial
// CPU arithmetic (an in-order fp32 sum for gemma4.c:600-601, serial double sums
// for lfm25.c:646-647 and maple.c:400-410, a serial double sum of squares in
// rmsnorm gemma4.c:425-428). A GPU reduces in parallel, so it cannot replay those
// roundings cheaply. Instead each value is computed in parallel together with a
// rigorous bound on its distance from the reference's serial result; a decision
// (a rounding to float, the top-k set and order) is taken on the GPU only when
// the bound proves it equals the reference's. Gemma logits carry a tight bound
// from their exact-order prefix sums; the rare values still contested are
// recomputed by replaying the reference's serial chain in the reference's order.
// Batches of 16+ tokens compute the gemma chains exactly instead (tiled kernel).
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_route_dev.h"
#include "zz_topk_wave.h"
#include <float.h>

// Prep: one workgroup per token. Gemma: the mean square is certified to round to
// the float the reference's serial double sum gives (gemma4.c:425-428), else that
// sum is replayed serially; then the router input xn = rmsnorm(x)*scale*D^-1/2
// (gemma4.c:591-593), unless there is no router (the dense branch, which routes
// every row to its one expert with weight 1 here). The expert input X (gemma: rmsnorm(x, pre_ffn_ln2),
// gemma4.c:763-764; lfm/maple: x) is quantised q8_0-style (q40.h:124-138), one
// 32-block per thread, with per-block integer sums; for tq2 the Sx total
// (tq2.h:98-108) is summed serially in the reference's order.
#define PREP_R 8           // float4 per thread: D <= 8192
__global__ __launch_bounds__(256) void zz_prep_kernel(ZzPrepArgs a) {
    const int s = blockIdx.x, D = a.D, tid = threadIdx.x, nb = D / ZZ_BLK, n4 = D / 4;
    const float *x = a.in + (size_t)s * D;
    __shared__ double red[4];
    __shared__ float xs_l[ZZ_MAXD / ZZ_BLK];
    __shared__ int xsum_l[ZZ_MAXD / ZZ_BLK];
    __shared__ float cert;
    // the row, its norm weights and router scale: every load issued first. Float4 i
    // of the row is value 4i..4i+3: block i/8, lane i%8 of the block's 8 lanes.
    const int R = (n4 + 255) >> 8;
    float4 xv[PREP_R], wv[PREP_R], sv[PREP_R];
#pragma unroll
    for (int k = 0; k < PREP_R; k++) {
        if (k >= R) break;
        const int i = min(tid + 256 * k, n4 - 1);
        xv[k] = *(const float4 *)(x + 4 * i);
        if (a.gemma) wv[k] = *(const float4 *)(a.pre_ln + 4 * i);
        if (a.gemma && a.router_scale) sv[k] = *(const float4 *)(a.router_scale + 4 * i);
    }
    if (a.route_eidx && tid == 0) {                // dense branch: one expert, weight 1
        a.route_eidx[s] = 0;
        a.route_ewt[s] = 1.0f;
    }
    float r = 1.0f;
    if (a.gemma) {
        double sq = 0.0;
#pragma unroll
        for (int k = 0; k < PREP_R; k++) {
            if (k >= R) break;
            if (tid + 256 * k < n4) {
                const float4 v = xv[k];
                sq += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
            }
        }
        sq = zz_block_sum(sq, red);
        // GPU: each term in <= R + 12 roundings; reference: D - 1 in order.
        // All terms are non-negative, so the exact sum is <= sq / (1 - g_m).
        const double m = (double)(R + 12);
        const double g = zz_gamma(D, ZZ_U64) + zz_gamma(m, ZZ_U64);
        const double b = g * sq / (1.0 - zz_gamma(m, ZZ_U64)) * 1.0000001 + 1e-300;
        const float lo = (float)((sq - b) / (double)D), hi = (float)((sq + b) / (double)D);
        if (tid == 0) {
            if (lo == hi) {
                cert = lo;
            } else {
                double t = 0.0;                    // serial replay, reference order
                for (int i = 0; i < D; i++) t += (double)x[i] * (double)x[i];
                cert = (float)(t / (double)D);
                atomicAdd(a.diag + 0, 1u);
            }
        }
        __syncthreads();
        r = 1.0f / sqrtf(cert + a.eps);
        if (a.router_scale) {                      // the router input (no router: no xn)
            const float rs = 1.0f / sqrtf((float)D);
#pragma unroll
            for (int k = 0; k < PREP_R; k++) {
                if (k >= R) break;
                const int i = tid + 256 * k;
                if (i < n4) {
                    const float4 v = xv[k], sc = sv[k];
                    *(float4 *)(a.xn + (size_t)s * D + 4 * i) =
                        make_float4((v.x * r) * (sc.x * rs), (v.y * r) * (sc.y * rs), (v.z * r) * (sc.z * rs),
                                    (v.w * r) * (sc.w * rs));
                }
            }
        }
    }
    // q8_0 of the expert input, 8 lanes per block (every lane of a wave takes part)
#pragma unroll
    for (int k = 0; k < PREP_R; k++) {
        if (k >= R) break;
        const int i = tid + 256 * k;
        float4 v = xv[k];
        if (a.gemma) {
            const float4 w = wv[k];
            v = make_float4((v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w);
        }
        float d;
        int qs;
        const unsigned pk = zz_quant8(v, &d, &qs);
        if (i < n4) {
            *(unsigned *)(a.xq + (size_t)s * D + 4 * i) = pk;
            if ((i & 7) == 0) {
                const int b = i >> 3;
                a.xs[(size_t)s * nb + b] = d;
                a.xsum[(size_t)s * nb + b] = qs;
                xs_l[b] = d;
                xsum_l[b] = qs;
            }
        }
    }
    if (a.xt) {
        __syncthreads();
        if (tid == 0) {
            double tot = 0.0;                      // tq2.h:101-106, serial
            for (int b = 0; b < nb; b++) tot += (double)xs_l[b] * (double)xsum_l[b];
            a.xt[s] = (float)tot;
        }
    }
}

#define ZZ_WAVE_LDS (4 * ZZ_TBUF > 8 * ZZ_DBUF ? 4 * ZZ_TBUF : 8 * ZZ_DBUF)   // bytes per wave
__global__ __launch_bounds__(256) void zz_logits_kernel(ZzLogitArgs a) {
    __shared__ __attribute__((aligned(16))) char buf[4 * ZZ_WAVE_LDS];
    const int s = blockIdx.y, e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= a.E) return;
    char *wb = buf + (threadIdx.x >> 6) * ZZ_WAVE_LDS;
    if (a.gating == ZZ_GATE_SOFTMAX_PES) {
        const size_t o = (size_t)s * a.E + e;
        zz_tight_wave<1, false>(a.router + (size_t)e * a.D, a.xn + (size_t)s * a.D, nullptr, nullptr,
                                1.0f, a.D, a.bias, e, (float *)wb, a.cen + o, a.bnd + o, a.E, nullptr);
    } else {
        zz_logit_wave_f64(a, s, e, (double *)wb);
    }
}

// -------------------------------------------------------------------------------
// Router logits for batches: the reference's own serial chains, exactly. One
// lane owns one (token, expert) pair and walks k = 0..D-1 in order:
//   gemma  v = v + fl(w_k * xn_k) in fp32, unfused (gemma4.c:600-601 as compiled:
//          vmulps then in-order vaddss);
//   lfm / maple  v = v + (double)w_k * x_k in double, then (float)v
//          (lfm25.c:646-647, maple.c:400-410);
//   ling   eight double accumulators by k % 8, combined pairwise (ling.c:722-727).
// The double product of two floats is exact, so v + (double)w * x rounds once and
// equals fma((double)w, (double)x, v): the double chains take one fma per element.
// A workgroup is TT tokens x 64 experts: wave w holds token s0 + w, lane l expert
// e0 + l. The 64 router rows are loaded from L2 straight into LDS in K chunks of KC
// (256 where D allows, else 64), double buffered, and each lane reads its own row as
// float4. The token's input is wave-uniform: a chunk sits in KC/16 VGPRs, 16 values
// each, lane l holding element l % 16 (every 16-lane row alike), and element j
// reaches all lanes by the DPP row broadcast (row_newbcast:j) folded into the
// multiply. The next chunk's loads (router rows and input) are issued before this
// chunk is summed and waited for after it: a chunk's 2 * KC VALU operations per wave
// are what hide the L2 / HBM latency, so KC = 64 (~200 ns of work) left every chunk
// waiting and KC = 256 does not. The chain is serial per lane, so the VALU time of
// one wave per SIMD (S * E / 64 waves) is the floor; LDS carries only the router
// operand.
#define LX_E 64
#define LX_WARM 3      // warm-up sectors per thread and operand
#define ZZ_WAIT_VM0 0x0F70   // s_waitcnt vmcnt(0), expcnt and lgkmcnt untouched (gfx9 fields)
// one wave moves 64 * B bytes from global memory to LDS: lane l's B bytes at g go to
// l_base + l * B (l_base wave-uniform); completion is counted by vmcnt
template <int B>
__device__ __forceinline__ void zz_load_lds(const float *g, float *l_base) {
    static_assert(B == 4 || B == 16, "4 or 16 bytes per lane");
    auto *l = (__attribute__((address_space(3))) void *)l_base;
    if constexpr (B == 16) __builtin_amdgcn_global_load_lds((const void *)g, l, 16, 0, 0);
    else __builtin_amdgcn_global_load_lds((const void *)g, l, 4, 0, 0);
}
// lane (l & ~15) + J's value of v, in every lane of its 16-lane row
template <int J>
__device__ __forceinline__ float zz_row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + J, 0xF, 0xF, false));
}
// 16 consecutive elements of one chain: w[J] (this lane's router row) times element
// J of the row-broadcast input xq; CH as below, acc[0] the chain (acc[J % 8] for ling)
typedef float zz_f4 __attribute__((ext_vector_type(4)));
template <int CH, int J = 0>
__device__ __forceinline__ void zz_chain16(float &vf, double *acc, const zz_f4 *w4, float xq) {
    if constexpr (J < 16) {
        const float xb = zz_row_bcast<J>(xq), w = w4[J / 4][J % 4];
        if constexpr (CH == 1) acc[0] = __builtin_fma((double)w, (double)xb, acc[0]);
        else acc[J % 8] = __builtin_fma((double)w, (double)xb, acc[J % 8]);
        zz_chain16<CH, J + 1>(vf, acc, w4, xq);
    }
}
// gemma's fp32 chain, 16 elements at a time: while the adds of group g run (in
// order, one rounding each, as the reference), the products of group g + 1 are
// formed between them, so the serial add chain never waits on its own multiply and
// every multiply fills an add's latency. The compiler pairs each multiply with its
// own add whatever the source order, so each step is written out: an unfused
// v_mul_f32 with the row broadcast of the next group's input (the same product as
// the reference's vmulps; operand order does not change a rounded product) and a
// v_add_f32 of this group's product. The leading s_nop 1 gives the two wait states a
// DPP read needs after a VALU write of its source.
#define ZZ_MA(J, QI, WI, PI) \
    "v_mul_f32_dpp %" #QI ", %[x], %" #WI " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n\t" \
    "v_add_f32 %[v], %[v], %" #PI "\n\t"
#define ZZ_MA4(J0, J1, J2, J3) \
    asm volatile("s_nop 1\n\t" ZZ_MA(J0, 0, 6, 10) ZZ_MA(J1, 1, 7, 11) ZZ_MA(J2, 2, 8, 12) ZZ_MA(J3, 3, 9, 13) \
                 : "=&v"(q[J0]), "=&v"(q[J1]), "=&v"(q[J2]), "=&v"(q[J3]), [v] "+v"(vf) \
                 : [x] "v"(xnext), "v"(w[J0]), "v"(w[J1]), "v"(w[J2]), "v"(w[J3]), \
                   "v"(p[J0]), "v"(p[J1]), "v"(p[J2]), "v"(p[J3]))
// vf += p[0..15] in order, and q[j] = w[j] * (element j of xnext's row broadcast)
__device__ __forceinline__ void zz_madd16(float &vf, const float *p, float *q, const float *w,
                                          float xnext) {
    ZZ_MA4(0, 1, 2, 3);
    ZZ_MA4(4, 5, 6, 7);
    ZZ_MA4(8, 9, 10, 11);
    ZZ_MA4(12, 13, 14, 15);
}
#undef ZZ_MA4
#undef ZZ_MA
template <int J = 0>
__device__ __forceinline__ void zz_prod16(float *p, const zz_f4 *w4, float xq) {
    if constexpr (J < 16) {
        p[J] = w4[J / 4][J % 4] * zz_row_bcast<J>(xq);
        zz_prod16<J + 1>(p, w4, xq);
    }
}
// CH: the chain kind -- 0 gemma's fp32 chain, 1 one double chain (lfm, maple),
// 2 ling's eight double accumulators; one instantiation each, so a chain carries only
// its own registers. KC: the K chunk (D % KC == 0). TT: tokens (waves) per workgroup,
// which share each staged router row: 8 where there are E / 64 >= 4 expert blocks
// (the grid still fills the chip at S = 512), else 4.
template <int CH, int KC, int TT>
__global__ __launch_bounds__(64 * TT, 1) void zz_logits_exact_kernel(ZzLogitArgs a) {
    constexpr int NT = 64 * TT;                       // threads
    const int tid = threadIdx.x, lane = tid & 63;
    const int s = blockIdx.x * TT + (tid >> 6), e0 = blockIdx.y * LX_E, e = e0 + lane, D = a.D;
    constexpr bool gem = CH == 0, grp = CH == 2;
    constexpr int NX = KC / 16;                       // input VGPRs per chunk
    const float *X = gem ? a.xn : a.x;
    // this lane's elements of the wave's input row (rows past the end read the last
    // row; not stored)
    const float *xrow = X + (size_t)min(s, a.S - 1) * D + (lane & 15);
    // gemma's harness logit offset, added after the chain: read now, not after it
    const float bz = gem && a.bias ? a.bias[min(e, a.E - 1)] : 0.0f;
    __shared__ __attribute__((aligned(16))) float ws_t[2][LX_E][KC + 4];
    // staging: wave w moves rows w, w + TT, ... of a chunk from L2 straight into LDS
    // (global_load_lds: lane l's KC/64 floats land at the row start + l * KC/16 bytes),
    // one row per instruction; rows past E repeat the last. Staged through registers,
    // each row would cost a VGPR load and an LDS write per lane, and the chunk's
    // register writes and LDS writes ran 1.7-1.9 us (of 34) slower at Gemma's S = 512.
    constexpr int RPW = LX_E / TT;
    const float *R = a.router;
    const float *drow[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++)
        drow[i] = R + (size_t)min(e0 + (tid >> 6) + TT * i, a.E - 1) * D + (KC / 64) * lane;
    auto stage = [&](int b, int k) {
#pragma unroll
        for (int i = 0; i < RPW; i++)
            zz_load_lds<KC / 16>(drow[i] + k, &ws_t[b][(tid >> 6) + TT * i][0]);
    };
    // the input of the chunk being summed and of the next one, in two register sets
    // that swap roles each chunk: a copy from one set to the other would be placed by
    // the compiler as soon as a register is free, early in the chunk, and wait there
    // for the next chunk's loads
    float xa[NX], xb[NX];
    stage(0, 0);
#pragma unroll
    for (int i = 0; i < NX; i++) xa[i] = xrow[16 * i];
    // L2 warm-up, issued behind chunk 0's loads: one dword per 64-byte sector of
    // (a) this XCD's share of the workgroup's router rows (workgroups are dealt to the
    // 8 XCDs round-robin, so those with the same blockIdx.x % 8 and blockIdx.y share
    // an L2: each takes every J-th sector) and (b) the workgroup's own input rows. A
    // layer's router and input are cold (the expert weights stream through every
    // cache between layers); warmed, the later chunks' loads hit L2 instead of each
    // chunk waiting out an HBM round trip. The values only pass through an empty asm.
    float warm[2 * LX_WARM];
    {
        const int nr = min(LX_E, a.E - e0), J = ((int)gridDim.x + 7) >> 3, j = blockIdx.x >> 3;
        const long ns = (long)nr * D / 16;
        const float *rb = R + (size_t)e0 * D;
        const int sx0 = blockIdx.x * TT, nx = min(TT, a.S - sx0);
        const float *xb = X + (size_t)sx0 * D;
        const int nsx = nx * D / 16;
#pragma unroll
        for (int r = 0; r < LX_WARM; r++) {
            const long sr = j + (long)J * (tid + NT * r);
            warm[r] = sr < ns ? rb[16 * sr] : 0.0f;
            const int sx = tid + NT * r;
            warm[LX_WARM + r] = sx < nsx ? xb[16 * sx] : 0.0f;
        }
    }
    __builtin_amdgcn_s_waitcnt(ZZ_WAIT_VM0);           // the staged rows have landed
    __syncthreads();
    float vf = 0.0f;
    double acc[grp ? 8 : 1];                          // grouped: ling.c's 8 accumulators
#pragma unroll
    for (int k = 0; k < (grp ? 8 : 1); k++) acc[k] = 0.0;
    int buf = 0;
    auto chunk = [&](int k0, const float (&xq)[NX], float (&xn)[NX]) {
        const int k1 = min(k0 + KC, D - KC);        // the last chunk reloads itself
        stage(buf ^ 1, k1);                          // free: every wave is past its reads
#pragma unroll
        for (int i = 0; i < NX; i++) xn[i] = xrow[k1 + 16 * i];
        // keep those loads here, a whole chunk ahead of their use (the scheduler
        // would otherwise sink each to just before it, and wait)
        __builtin_amdgcn_sched_barrier(0);
        const float *wr = ws_t[buf][lane];
        if constexpr (gem) {
            zz_f4 w4[2][4];                         // the next group's row and the one after
            float p[16], q[16];
#pragma unroll
            for (int r = 0; r < 4; r++) w4[0][r] = *(const zz_f4 *)(wr + 4 * r);
            zz_prod16(p, w4[0], xq[0]);
#pragma unroll
            for (int r = 0; r < 4; r++) w4[1][r] = *(const zz_f4 *)(wr + 16 + 4 * r);
#pragma unroll
            for (int i = 0; i < NX; i++) {          // element k0 + 16i + j
                if (i + 1 < NX) {
                    float w[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) w[j] = w4[(i + 1) & 1][j / 4][j % 4];
                    if (i + 2 < NX) {
#pragma unroll
                        for (int r = 0; r < 4; r++) w4[i & 1][r] = *(const zz_f4 *)(wr + 16 * (i + 2) + 4 * r);
                    }
                    zz_madd16(vf, p, q, w, xq[i + 1]);
#pragma unroll
                    for (int j = 0; j < 16; j++) p[j] = q[j];
                } else {
#pragma unroll
                    for (int j = 0; j < 16; j++) vf = vf + p[j];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NX; i++) {          // element k0 + 16i + j: acc j % 8
                zz_f4 w4[4];
#pragma unroll
                for (int r = 0; r < 4; r++) w4[r] = *(const zz_f4 *)(wr + 16 * i + 4 * r);
                zz_chain16<CH>(vf, acc, w4, xq[i]);
            }
        }
        __builtin_amdgcn_s_waitcnt(ZZ_WAIT_VM0);
        __syncthreads();
        buf ^= 1;
    };
    int k0 = 0;
    for (; k0 + 2 * KC <= D; k0 += 2 * KC) {
        chunk(k0, xa, xb);
        chunk(k0 + KC, xb, xa);
    }
    if (k0 < D) chunk(k0, xa, xb);
#pragma unroll
    for (int r = 0; r < 2 * LX_WARM; r++) asm volatile("" ::"v"(warm[r]));
    if (s < a.S && e < a.E) {
        const size_t o = (size_t)s * a.E + e;
        if constexpr (gem) {
            if (a.bias) vf = vf + bz;              // harness logit offset, after the dot
            a.cen[o] = (double)vf;
        } else {
            double vd = acc[0];
            if constexpr (grp)
                vd = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
            a.cen[o] = (double)(float)vd;
        }
        a.bnd[o] = 0.0;                             // exact: no interval
    }
}

template <int KC, int TT>
static void zz_launch_logits_exact_tt(const ZzLogitArgs &b, int S, hipStream_t st) {
    const dim3 g((S + TT - 1) / TT, (b.E + LX_E - 1) / LX_E), t(64 * TT);
    if (b.gating == ZZ_GATE_SOFTMAX_PES) hipLaunchKernelGGL((zz_logits_exact_kernel<0, KC, TT>), g, t, 0, st, b);
    else if (b.gating == ZZ_GATE_GROUPED) hipLaunchKernelGGL((zz_logits_exact_kernel<2, KC, TT>), g, t, 0, st, b);
    else hipLaunchKernelGGL((zz_logits_exact_kernel<1, KC, TT>), g, t, 0, st, b);
}
template <int KC>
static void zz_launch_logits_exact(const ZzLogitArgs &b, int S, hipStream_t st) {
    if (b.E >= 4 * LX_E) zz_launch_logits_exact_tt<KC, 8>(b, S, st);
    else zz_launch_logits_exact_tt<KC, 4>(b, S, st);
}

// Top-k gating, one wave per token (zz_topk_wave.h), four tokens per workgroup.
__global__ __launch_bounds__(256) void zz_topk_kernel(ZzTopkArgs a, int S) {
    extern __shared__ __attribute__((aligned(16))) char tk_lds[];
    const int w = threadIdx.x >> 6, s = blockIdx.x * 4 + w;
    if (s >= S) return;
    zz_topk_wave_any(a, s, tk_lds + w * zz_topk_wave_bytes(a.E));
}

// -------------------------------------------------------------------------------
// Dispatch, one workgroup of 1024 threads. Each expert gets a bitmask over tokens;
// a pair's place in its expert's list is the expert's start plus the number of
// earlier tokens that chose it (a popcount) -- the stable counting sort that gives
// exactly rows[] of gemma4.c:779-786, ascending tokens. The smallest pair index
// of each expert orders the union as first-seen (gemma4.c:756-761). Also emits
// the FFN work list: per expert in union order, chunks of at most `tch` pairs.
// inclusive prefix sum over a wave by DPP: shifts within each 16-lane row by 1, 2,
// 4, 8 (lanes shifted in from outside the row add 0), then the rows' running totals
// (row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, row_bcast:31 the
// total of rows 0-1 to rows 2 and 3). 32 or 64 bits (64: both halves move, one add).
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned zz_dpp_u32(unsigned v) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned long long zz_dpp_u64(unsigned long long v) {
    return ((unsigned long long)zz_dpp_u32<CTRL, ROWS>((unsigned)(v >> 32)) << 32) | zz_dpp_u32<CTRL, ROWS>((unsigned)v);
}
template <typename T>
__device__ __forceinline__ T zz_wave_incl_scan(T x) {
    if constexpr (sizeof(T) == 8) {
        x += zz_dpp_u64<0x111, 0xF>(x);
        x += zz_dpp_u64<0x112, 0xF>(x);
        x += zz_dpp_u64<0x114, 0xF>(x);
        x += zz_dpp_u64<0x118, 0xF>(x);
        x += zz_dpp_u64<0x142, 0xA>(x);
        x += zz_dpp_u64<0x143, 0xC>(x);
    } else {
        x += zz_dpp_u32<0x111, 0xF>(x);
        x += zz_dpp_u32<0x112, 0xF>(x);
        x += zz_dpp_u32<0x114, 0xF>(x);
        x += zz_dpp_u32<0x118, 0xF>(x);
        x += zz_dpp_u32<0x142, 0xA>(x);
        x += zz_dpp_u32<0x143, 0xC>(x);
    }
    return x;
}

// exclusive prefix sum over the threads of a workgroup (up to 1024; tmp: 16 entries
// of LDS): the wave scans, then each thread adds the totals of the waves before its
// own, all 15 read at once (a loop over them, one read after another, cost the last
// wave ~0.5 us per scan). Two barriers.
template <typename T>
__device__ __forceinline__ T zz_block_excl_scan_t(T v, T *tmp) {
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const T x = zz_wave_incl_scan(v);
    if (l == 63) tmp[w] = x;
    __syncthreads();
    T base = 0;
#pragma unroll
    for (int q = 0; q < 15; q++) base += q < w ? tmp[q] : (T)0;
    __syncthreads();                           // tmp is free again for the next scan
    return base + x - v;
}
__device__ __forceinline__ int zz_block_excl_scan(int v, int *tmp) {
    return (int)zz_block_excl_scan_t<unsigned>((unsigned)v, (unsigned *)tmp);
}

__device__ __forceinline__ unsigned zz_uni(unsigned v) { return (unsigned)__builtin_amdgcn_readfirstlane((int)v); }

// exclusive prefix sum of a 64-bit value over the workgroup (tmp: 16 entries of LDS)
__device__ __forceinline__ unsigned long long zz_block_excl_scan64(unsigned long long v, unsigned long long *tmp) {
    return zz_block_excl_scan_t<unsigned long long>(v, tmp);
}

#define DP_T 1024                     // threads
#define DP_PT 8                       // pairs per thread: S*K <= 8192 = DP_T * DP_PT
// One workgroup: the per-expert token bitmasks give each expert's count, its pairs'
// positions (a stable counting sort by expert, gemma4.c:779-786) and its first pair;
// the union order is the order of first pairs (gemma4.c:756-761), read off a bitmap
// over the pairs by prefix popcounts.
// LDS: mask and word prefixes [E][W] (W = S/32 words), first-pair bitmap [P/32],
// pair experts [P].
__global__ __launch_bounds__(DP_T) void zz_dispatch_kernel(ZzDispatchArgs a) {
    extern __shared__ unsigned dsm[];
    __shared__ int cnt[ZZ_MAXE], start[ZZ_MAXE], first[ZZ_MAXE], order[ZZ_MAXE], tmp[16];
    __shared__ int xcost[ZZ_MAXE], xof[ZZ_MAXE], xjb[ZZ_MAXE], xslot[9], xrank[ZZ_MAXE], xrc[ZZ_MAXE];
    __shared__ unsigned xload[8], uload[8];
    __shared__ unsigned long long tmp64[16];
    __shared__ int xtotal;
    __shared__ int fbase[DP_PT * DP_T / 32];      // first pairs before each bitmap word
    const int P = a.P, E = a.E, K = a.K, S = P / K, W = (S + 31) / 32, PW = (P + 31) / 32, t = threadIdx.x;
    unsigned *mask = dsm, *wpre = dsm + E * W, *fb = wpre + E * W;
    int *pe = (int *)(fb + PW);                  // pair -> expert
    for (int i = t; i < E * W; i += DP_T) mask[i] = 0u;
    for (int i = t; i < PW; i += DP_T) fb[i] = 0u;
    // every pair's expert and weight in registers first: one round of loads
    int ev[DP_PT];
    float wv[DP_PT];
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = min(t + DP_T * k, P - 1);
        const int e = a.eidx[p];
        ev[k] = e < 0 || e >= E ? 0 : e;            // never index past the expert tables
        wv[k] = a.ewt[p];
    }
#pragma unroll
    for (int k = 0; k < DP_PT; k++)
        if (t + DP_T * k < P) pe[t + DP_T * k] = ev[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = t + DP_T * k, s = p / K;
        if (p < P) atomicOr(&mask[ev[k] * W + (s >> 5)], 1u << (s & 31));
    }
    __syncthreads();
    // per expert: word prefix counts, the count, and the first pair that routes to
    // it (its lowest token, that token's slot holding e)
    for (int e = t; e < E; e += DP_T) {
        int run = 0, s0 = -1;
        for (int w = 0; w < W; w++) {
            const unsigned m = mask[e * W + w];
            wpre[e * W + w] = run;
            if (s0 < 0 && m) s0 = 32 * w + __ffs(m) - 1;
            run += __popc(m);
        }
        cnt[e] = run;
        int f = 0x7fffffff;
        if (s0 >= 0) {
            for (int j = K - 1; j >= 0; j--)
                if (pe[s0 * K + j] == e) f = s0 * K + j;
            atomicOr(&fb[f >> 5], 1u << (f & 31));
        }
        first[e] = f;
    }
    const int st = zz_block_excl_scan(t < E ? cnt[t] : 0, tmp);   // its barrier orders the above
    if (t < E) start[t] = st;
    // union rank of each present expert: first pairs below its own
    const int fw = t < PW ? __popc(fb[t]) : 0;
    const int fpre = zz_block_excl_scan(fw, tmp);
    if (t < PW) fbase[t] = fpre;
    __syncthreads();
    const bool present = t < E && cnt[t] != 0;
    if (present) {
        const int f = first[t];
        order[fbase[f >> 5] + __popc(fb[f >> 5] & ((1u << (f & 31)) - 1u))] = t;
    }
    if (t < 8) uload[t] = 0;
    const int nu = __syncthreads_count(present);
    const int ce = t < nu ? cnt[order[t]] : 0;
    const int nit = (ce + a.tch - 1) / a.tch;
    const int i0 = zz_block_excl_scan(nit, tmp);
    // XCD placement of the work items. Workgroup g of an FFN launch runs on XCD g % 8
    // and each XCD has its own L2, so all items of one expert go to one XCD, where
    // they run back to back and read the expert's weights from HBM once. An expert's
    // load is its weight stream (wcost) plus the token columns of its items (16 per
    // started tile of 16, 4 for an item of <= 4 tokens). The union is placed in batches
    // of 8 consecutive experts (union order: first seen, which puts the popular experts
    // first): the batch's costliest expert goes to the least loaded XCD, the next to the
    // next, and so on (ties to the lower expert and XCD). A batch's experts land on 8
    // different XCDs and each XCD runs its items in union order, which keeps heavy and
    // light experts interleaved in time. (Placing expert by expert on the least loaded
    // XCD balanced as well, max/mean load 1.019 against 1.018 over eight Zipf routings,
    // but took 8 µs of dependent steps; dealing experts in a fixed order, or running each
    // XCD's heavy experts first, measured slower.) Item slot j*8 + x is XCD x's j-th
    // item. Without an expert of several items, or when the placement's costliest XCD
    // would carry more than union order's, the items keep union order, item i on XCD i % 8.
    int cost = 0;
    if (t < nu) {
        cost = a.wcost;
        for (int c = 0; c < nit; c++) {
            const int n = min(a.tch, ce - c * a.tch), cols = n <= 4 ? 4 : 16 * ((n + 15) >> 4);
            cost += cols;
            atomicAdd(&uload[(i0 + c) & 7], (unsigned)(a.wcost + cols));   // the same in union order
        }
        xcost[t] = cost;
    }
    const int nm = __syncthreads_count(t < nu && nit > 1);
    if (nm > 0) {
        // each expert's rank within its batch (cost descending, then union order); the
        // batch's experts listed by rank, with their costs
        if (t < nu) {
            const int b0 = t & ~7, my = xcost[t];
            int rk = 0;
#pragma unroll
            for (int j = b0; j < b0 + 8; j++) {         // all 8 reads at once
                const int cj = j < nu ? xcost[j] : -1;
                rk += (cj > my) | ((cj == my) & (j < t));
            }
            xrank[b0 + rk] = t;
            xrc[b0 + rk] = my;
        }
        __syncthreads();
        if (t < 16) {
            // Lanes x and x + 8 (one DPP row) keep XCD x's load; the key (load << 3) | x
            // orders the XCDs by load, then x, and the rotations of the row by 1..7 lanes
            // bring every other XCD's key. The XCD of rank r by load takes the batch's
            // expert of rank r by cost.
            const int x = t & 7;
            unsigned key = (unsigned)x;
            for (int b0 = 0; b0 < nu; b0 += 8) {
                int rx = 0;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x121, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x122, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x123, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x124, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x125, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x126, 0xF, 0xF, false) < key;
                rx += (unsigned)__builtin_amdgcn_update_dpp(0, (int)key, 0x127, 0xF, 0xF, false) < key;
                if (b0 + rx < nu) {
                    key += (unsigned)xrc[b0 + rx] << 3;
                    if (t < 8) xof[xrank[b0 + rx]] = x;
                }
            }
            if (t < 8) xload[x] = key >> 3;
        }
    }
    // positions of the pairs (a stable counting sort), each thread its own pairs,
    // with the sorted lists written straight to their positions
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = t + DP_T * k;
        if (p < P) {
            const int e = ev[k], s = p / K, w = s >> 5, bit = s & 31;
            const int pos = start[e] + wpre[e * W + w] + __popc(mask[e * W + w] & ((1u << bit) - 1u));
            a.ppos[p] = pos;
            a.ptok[pos] = s;
            a.pslot[pos] = p - s * K;
            a.pwt[pos] = wv[k];
        }
    }
    __syncthreads();                             // wave 0's placement is done
    // slot of each expert's first item: the items of earlier experts on its XCD, from
    // one exclusive scan of per-XCD item counts packed a byte per XCD
    if (t == nu - 1) xtotal = i0 + nit;                 // all items
    if (nu == 0 && t == 0) xtotal = 0;
    // xof is written only by the placement (nm > 0); union order needs no XCD here
    const int xe = t < nu && nm > 0 ? xof[t] : 0;
    const unsigned long long cnt8 = t < nu ? (unsigned long long)min(nit, 255) << (8 * xe) : 0ull;
    const unsigned long long pre8 = zz_block_excl_scan64(cnt8, tmp64);
    if (t < nu) xjb[t] = (int)((pre8 >> (8 * xe)) & 255u);
    if (t == DP_T - 1) {
        const unsigned long long tot8 = pre8 + cnt8;
        int mx = 0, sum = 0;
        for (int x = 0; x < 8; x++) {
            const int c = (int)((tot8 >> (8 * x)) & 255u);
            mx = max(mx, c);
            sum += c;
            xslot[x] = c;
        }
        // a count above 255 carries into the next byte (or out) and breaks the sum.
        // The placement is kept when its costliest XCD carries no more than union
        // order's would, where an expert pays its weight stream on every XCD that
        // runs one of its items. (A dense MLP's one expert of 8 items, or fewer
        // experts than XCDs, would leave XCDs idle: union order.)
        unsigned pmax = 0, umax = 0;
        for (int x = 0; nm > 0 && x < 8; x++) {
            pmax = max(pmax, xload[x]);
            umax = max(umax, uload[x]);
        }
        xslot[8] = sum == xtotal && nm > 0 && pmax <= umax ? mx : 1 << 30;
    }
    __syncthreads();
    // a placement past the grid's slots per XCD (never at realistic routings) or a
    // costlier one: items in union order instead, item i on XCD i % 8, which always fits
    const int ms = xslot[8];
    const bool placed = ms <= a.xslots;
    if (t < nu) {
        const int e = order[t];
        a.uniq[t] = e;
        a.uoff[t] = start[e];
        a.ucnt[t] = ce;
        for (int c = 0; c < nit; c++) {
            ZzItem it;
            it.e = e;
            it.u = t;
            it.p0 = start[e] + c * a.tch;
            it.n = min(a.tch, ce - c * a.tch);
            a.items[placed ? (xjb[t] + c) * 8 + xof[t] : i0 + c] = it;
        }
    }
    const int total = placed ? 8 * ms : (i0 + nit + 7) / 8 * 8;     // (unplaced: read at t = nu - 1)
    if (placed) {
        for (int i = t; i < 8 * ms; i += DP_T)
            if (i / 8 >= xslot[i & 7]) a.items[i].n = 0;
    }
    if (t == nu - 1 || (nu == 0 && t == 0)) {
        a.meta[0] = nu;
        a.meta[1] = total;
        for (int i = i0 + nit; !placed && i < total; i++) a.items[i].n = 0;
    }
}

// ------------------------------------------------------------------ launchers
int zz_launch_prep(const ZzPrepArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_prep_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_logits(const ZzLogitArgs &a, int S, hipStream_t st) {
    if (S >= a.exact_min_s && a.D % 64 == 0) {
        ZzLogitArgs b = a;
        b.S = S;
        if (a.D % 256 == 0) zz_launch_logits_exact<256>(b, S, st);
        else zz_launch_logits_exact<64>(b, S, st);
    } else {
        hipLaunchKernelGGL(zz_logits_kernel, dim3((a.E + 3) / 4, S), dim3(256), 0, st, a);
    }
    return hipGetLastError() == hipSuccess;
}

int zz_launch_topk(const ZzTopkArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_topk_kernel, dim3((S + 3) / 4), dim3(256), 4 * zz_topk_wave_bytes(a.E), st, a, S);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dispatch(const ZzDispatchArgs &a, hipStream_t st) {
    const int W = (a.P / a.K + 31) / 32, PW = (a.P + 31) / 32;
    const size_t lds = sizeof(unsigned) * (2 * (size_t)a.E * W + PW) + 4 * (size_t)a.P;
    hipLaunchKernelGGL(zz_dispatch_kernel, dim3(1), dim3(DP_T), lds, st, a);
    return hipGetLastError() == hipSuccess;
}

// the routers' expf on n values (a diagnostic: the device's bits against the host's)
__global__ void __launch_bounds__(256) zz_expf_kernel(const float *x, float *y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        y[i] = zz_expf(x[i]);
}

int zz_launch_expf(const float *x, float *y, int64_t n, hipStream_t st) {
    const int64_t want = (n + 255) / 256;
    hipLaunchKernelGGL(zz_expf_kernel, dim3((unsigned)(want < 8192 ? want : 8192)), dim3(256), 0, st, x, y, n);
    return hipGetLastError() == hipSuccess;
}
