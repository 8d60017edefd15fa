// zz_topk_wave.h -- certified top-k gating of one token by one wave.
//
// Each expert's selection score is known as an interval [lo, hi] that contains
// the reference's value (zz_route_dev.h). The top k by the reference's order
// (value descending, index ascending: the strict '>' insertion of
// gemma4.c:604-607, lfm25.c:650-659, maple.c:588-594) are fixed without any
// block-wide pass over all experts:
//   1. keys (lo rounded down to float, index) in registers, EPL experts per lane;
//      the k-th largest of the 64 lane maxima is <= the k-th largest key;
//   2. the few keys at or above it are compacted to LDS and ranked exactly: lk,
//      a float lower bound of the k-th largest lo (rounding down is monotone);
//   3. candidates are the experts with hi >= lk -- a superset of the top k;
//   4. a candidate whose interval meets another candidate's is contested; gemma
//      replays contested logits with the reference's serial fp32 chain
//      (gemma4.c:600-601). lfm/maple/ling scores are exact points: their logits
//      are exact floats and the sigmoid uses glibc's expf bit for bit (zz_expf.h);
//   5. candidates are ranked by centre (disjoint intervals order as their
//      values do; replayed ones are exact; equal values go to the lower expert,
//      counted in diag[3]), and the gate weights are formed.
// A register-only fast path settles the common case first: K rounds of a wave
// maximum give the K largest keys, which are the answer, in order, when no other
// expert's interval reaches the K-th lower bound and the K intervals are disjoint.
#pragma once
#include "zz_expf.h"
#include "zz_route_dev.h"

struct ZzTopkWaveHdr {
    unsigned long long etab[32];    // expf's table (zz_exp2_tab32), staged with the inputs
    unsigned long long lmax[64];
    unsigned long long lk;
    int idx[ZZ_MAXK];           // the result: expert of each slot
    float topv[ZZ_MAXK];
    float wt[ZZ_MAXK];          // the result: gate weight of each slot
};
// LDS of one wave: the header, then u64 ck[E], double clo[E], chi[E], int ci[E]
__host__ __device__ inline size_t zz_topk_wave_bytes(int E) {
    return (sizeof(ZzTopkWaveHdr) + (size_t)E * (8 + 8 + 8 + 4) + 15) & ~(size_t)15;
}

__device__ __forceinline__ unsigned zz_ord32(float f) {          // order-preserving bits
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float zz_unord32(unsigned u) {
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ float zz_round_down(double v) {
    float f = (float)v;
    if ((double)f > v) f = nextafterf(f, -INFINITY);
    return f;
}
// Wave maximum of an unsigned value through DPP: swaps within quads, the half-row
// and row mirrors, then the row broadcasts (lane 15 into rows 1 and 3, lane 31 into
// rows 2 and 3); lane 63 ends with the maximum. Lanes a step leaves out keep 0.
__device__ __forceinline__ unsigned zz_wave_umax(unsigned v) {
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));  // row_bcast:15
    v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));  // row_bcast:31
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

// a double held by lane q (q uniform)
__device__ __forceinline__ double zz_readlane_f64(double v, int q) {
    const unsigned long long u = __double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(u & 0xffffffffu), q);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(u >> 32), q);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ unsigned long long zz_lane_lt_mask() {
    const int l = threadIdx.x & 63;
    return l ? (~0ull >> (64 - l)) : 0ull;
}

// expf with the wave's LDS copy of the table: read from device memory at the point
// of use, the table cost a memory round trip in the middle of every top-k
__device__ __forceinline__ float zz_expf_lds(float x, const unsigned long long *etab) {
    return zz_expf_tab(x, [etab](int i) { return (uint64_t)etab[i]; });
}

// sigmoid score of an exact float logit, as lfm25.c:654 / ling.c:731 form it:
// 1.0f / (1.0f + expf(-v)), bit for bit
__device__ __forceinline__ float zz_sigmoid_score(double logit, const unsigned long long *etab) {
    const float v = (float)logit;
    return 1.0f / (1.0f + zz_expf_lds(-v, etab));
}

// The reference's gemma logit of expert e for router input xn: in-order fp32 sum
// of the rounded products, then + bias. Every lane computes the same chain.
__device__ float zz_gemma_chain(const float *w, const float *xn, int D, const float *bias, int e) {
    const int l = threadIdx.x & 63;
    float v = 0.0f;
    for (int i0 = 0; i0 < D; i0 += 64) {                     // D % 64 == 0
        const float p = w[i0 + l] * xn[i0 + l];
        const int pi = __float_as_int(p);
#pragma unroll
        for (int k = 0; k < 64; k++) v = v + __int_as_float(__builtin_amdgcn_readlane(pi, k));
    }
    if (bias) v = v + bias[e];
    return v;
}

// Gate weights of a selected set (the header's idx / topv): lane l < K holds slot l's
// centre cj and scale pj. Per slot in parallel, their sum serially in slot order as the
// reference adds them, then each slot's normalisation. write: store eidx, ewt, topv.
__device__ __forceinline__ void zz_topk_gates(const ZzTopkArgs &a, int s, ZzTopkWaveHdr &h, double cj, float pj,
                                              bool write) {
    const int K = a.K, l = threadIdx.x & 63;
    const bool sig = a.gating == ZZ_GATE_SIGMOID_BIAS || a.gating == ZZ_GATE_GROUPED;
    const int ej = l < K ? h.idx[l] : 0;
    float wj = 0.0f;
    if (l < K) wj = sig ? zz_sigmoid_score(cj, h.etab) : zz_expf_lds(h.topv[l] - h.topv[0], h.etab);
    float sum = 0.0f;
    for (int j = 0; j < K; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj), j));
    if (l < K) {
        float out;
        if (a.gating == ZZ_GATE_SOFTMAX_PES) {                     // gemma4.c:609-612
            out = (wj / sum) * pj;
        } else if (a.gating == ZZ_GATE_GROUPED) {                  // ling.c:783-788
            float t = wj;
            if (a.norm_topk && K > 1) t /= (sum + 1e-20f);
            out = t * a.routed_scaling;
        } else if (sig) {                                          // lfm25.c:661-667
            float t = wj;
            if (a.norm_topk) t /= (sum + 1e-6f);
            out = t * a.routed_scaling;
        } else {                                                   // maple.c:596-600
            float t = wj;
            if (a.norm_topk) t /= (sum + 1e-20f);
            out = t;
        }
        h.wt[l] = out;
        if (write) {
            a.eidx[(size_t)s * K + l] = ej;
            a.ewt[(size_t)s * K + l] = out;
            if (a.topv) a.topv[(size_t)s * K + l] = h.topv[l];
        }
    }
    zz_wave_sync_lds();
}

// write: store the routing outputs (eidx, ewt, topv, counters); gates: form the gate
// weights now (else only the selection, the header's idx and topv: the caller forms
// them later with zz_topk_wave_gates, from the same LDS)
template <int EPL>
__device__ void zz_topk_wave(const ZzTopkArgs &a, int s, char *lds, bool write, bool gates) {
    ZzTopkWaveHdr &h = *(ZzTopkWaveHdr *)lds;
    const int E = a.E, K = a.K, l = threadIdx.x & 63;
    unsigned long long *ck = (unsigned long long *)(lds + sizeof(ZzTopkWaveHdr));
    double *clo = (double *)(ck + E), *chi = clo + E;
    int *ci = (int *)(chi + E);
    const double *cen = a.cen + (size_t)s * E, *bnd = a.bnd + (size_t)s * E;
    const bool sig = a.gating == ZZ_GATE_SIGMOID_BIAS || a.gating == ZZ_GATE_GROUPED;
    const unsigned long long ltm = zz_lane_lt_mask();

    // intervals and keys; every load is issued before any is used (the expf table
    // too: lane l moves its 32-bit word to the header's copy)
    const unsigned tabw = ((const unsigned *)zz_exp2_tab32)[l];
    double cv[EPL], bv[EPL];
    float bi[EPL], pv[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = min(l + 64 * j, E - 1);
        cv[j] = cen[e];
        bv[j] = sig ? 0.0 : bnd[e];
        bi[j] = sig && a.bias ? a.bias[e] : 0.0f;
        pv[j] = a.gating == ZZ_GATE_SOFTMAX_PES ? a.pes[e] : 1.0f;    // the gate's scale, read now
    }
    ((unsigned *)h.etab)[l] = tabw;
    zz_wave_sync_lds();
    double lo[EPL], hi[EPL];
    unsigned long long key[EPL];
    int width = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = l + 64 * j;
        if (sig) {
            // the reference's selection score s + bias, exactly (lfm25.c:654-655)
            const float sg = zz_sigmoid_score(cv[j], h.etab);
            const float sel = a.bias ? sg + bi[j] : sg;
            lo[j] = hi[j] = (double)sel;
        } else {
            lo[j] = cv[j] - bv[j];
            hi[j] = cv[j] + bv[j];
            width |= bv[j] > 0.0;
        }
        if (!(lo[j] == lo[j])) lo[j] = -INFINITY;            // NaN scores never win
        if (!(hi[j] == hi[j])) hi[j] = -INFINITY;
        key[j] = e < E ? ((unsigned long long)zz_ord32(zz_round_down(lo[j])) << 32) |
                             (0xffffffffu - (unsigned)e)
                       : 0ull;
        if (e >= E) lo[j] = hi[j] = -INFINITY;
    }
    width = __ballot(width) != 0ull;
    int ties = 0;                                        // an exact tie decided by index

    // Grouped router (ling.c:734-760), on the exact selection scores: each group's
    // score is the float sum of its two best, the best topk_group groups are kept by
    // the reference's strict-'>' insertion (score desc, group asc; a score of -inf
    // or NaN is never kept), and the experts of the other groups leave the running.
    if (a.gating == ZZ_GATE_GROUPED) {
        const int NG = a.n_group, TG = a.topk_group, EG = E / NG;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int e = l + 64 * j;
            if (e < E) clo[e] = lo[j];
        }
        zz_wave_sync_lds();
        float gs = -INFINITY;
        if (l < NG) {
            float a1 = -INFINITY, a2 = -INFINITY;
            for (int i = 0; i < EG; i++) {
                const float x = (float)clo[l * EG + i];
                if (x > a1) { a2 = a1; a1 = x; } else if (x > a2) a2 = x;
            }
            gs = EG > 1 ? a1 + a2 : a1;
        }
        const bool valid = l < NG && gs > -INFINITY;
        int rk = 0;
        for (int q = 0; q < NG; q++) {
            const float gq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs), q));
            rk += (gq > gs) | ((gq == gs) & (q < l));
        }
        const unsigned long long live = __ballot(valid && rk < TG);
        // a tie across the boundary: the last kept group's score equals the first dropped one's
        const unsigned long long at = __ballot(valid && rk == TG - 1), nx = __ballot(valid && rk == TG);
        if (at && nx) {
            const float g0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs), (int)__ffsll((long long)at) - 1));
            const float g1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs), (int)__ffsll((long long)nx) - 1));
            ties |= g0 == g1;
        }
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const int e = l + 64 * j;
            if (e < E && !((live >> (e / EG)) & 1ull)) {
                lo[j] = hi[j] = -INFINITY;
                key[j] = 0ull;
            }
        }
        zz_wave_sync_lds();                              // clo / chi are reused below
    }

    // Fast path, registers only: the K largest keys by K rounds of a wave maximum.
    // It stands when no other expert's hi reaches the K-th key's lo (the K are the
    // set) and, in key order, every interval lies strictly above all later ones (the
    // key order is the true order). Otherwise the general passes below decide.
    bool fast = false;
    {
        // key order = (float part desc, expert asc): a DPP wave maximum of the float
        // part, then the lowest expert holding it by ballot (e = lane + 64 j)
        unsigned kh[EPL];
#pragma unroll
        for (int j = 0; j < EPL; j++) kh[j] = (unsigned)(key[j] >> 32);
        int sel_e = 0;                                     // lane r < K: the r-th key's expert
        unsigned top = 0u;
        for (int r = 0; r < K; r++) {
            unsigned m = 0u;
#pragma unroll
            for (int j = 0; j < EPL; j++) m = kh[j] > m ? kh[j] : m;
            m = zz_wave_umax(m);
            int e = -1;
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const unsigned long long b = __ballot(kh[j] == m);
                if (e < 0 && b) e = (int)__ffsll((long long)b) - 1 + 64 * j;
            }
            if (l == (e & 63)) kh[e >> 6] = 0u;            // taken (valid keys are > 0)
            if (l == r) sel_e = e;
            top = m;
        }
        const double lk0 = (double)zz_unord32(top);
        int nc = 0;
#pragma unroll
        for (int j = 0; j < EPL; j++) nc += __popcll(__ballot(l + 64 * j < E && hi[j] >= lk0));
        if (top != 0u && nc == K) {
            // lane r < K fetches its expert's interval from the owning lane
            double slo = 0.0, shi = 0.0;
            const int own = sel_e & 63, jj = sel_e >> 6;
#pragma unroll
            for (int j = 0; j < EPL; j++) {
                const double a = __shfl(lo[j], own, 64), b = __shfl(hi[j], own, 64);
                if (jj == j) { slo = a; shi = b; }
            }
            // every interval strictly above all later ones: hi of rank q < lo of each
            // earlier rank, i.e. a suffix maximum of hi against lo
            double later = -INFINITY;
            for (int q = K - 1; q >= 1; q--) {
                const double hq = zz_readlane_f64(shi, q);
                if (l < q) later = hq > later ? hq : later;
            }
            const bool ok = l >= K - 1 || later < slo;
            if (__ballot(!ok) == 0ull) {
                fast = true;
                if (l < K) {
                    h.idx[l] = sel_e;
                    h.topv[l] = (float)(0.5 * (slo + shi));
                }
            }
        }
    }

    if (!fast) {
    // 1. the k-th largest lane maximum (keys are distinct; empty lanes hold 0)
    unsigned long long mk = 0ull;
#pragma unroll
    for (int j = 0; j < EPL; j++) mk = key[j] > mk ? key[j] : mk;
    h.lmax[l] = mk;
    if (l < K) {
        h.idx[l] = l;                                         // valid ids whatever happens
        h.topv[l] = 0.0f;
    }
    zz_wave_sync_lds();
    int r = 0;
#pragma unroll 16
    for (int q = 0; q < 64; q++) r += h.lmax[q] > mk;
    if (r == K - 1) h.lk = mk;
    zz_wave_sync_lds();
    const unsigned long long thr = h.lk;

    // 2. exact k-th largest key among the keys >= thr
    int c = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const bool p = key[j] >= thr && key[j] != 0ull;
        const unsigned long long m = __ballot(p);
        if (p) ck[c + __popcll(m & ltm)] = key[j];
        c += __popcll(m);
    }
    zz_wave_sync_lds();
    for (int i = l; i < c; i += 64) {
        const unsigned long long k = ck[i];
        int rk = 0;
        for (int q = 0; q < c; q++) rk += ck[q] > k;
        if (rk == K - 1) h.lk = k;
    }
    zz_wave_sync_lds();
    const double lk = (double)zz_unord32((unsigned)(h.lk >> 32));

    // 3. candidates: hi >= lk
    int nc = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const bool p = l + 64 * j < E && hi[j] >= lk;
        const unsigned long long m = __ballot(p);
        if (p) {
            const int pos = nc + __popcll(m & ltm);
            ci[pos] = l + 64 * j;
            clo[pos] = lo[j];
            chi[pos] = hi[j];
        }
        nc += __popcll(m);
    }
    zz_wave_sync_lds();

    // 4. contested candidates. Only gemma's bounded logits have width: exact values
    // can only tie, which the index order below resolves as the reference does
    int any = 0;
    if (width && a.gating == ZZ_GATE_SOFTMAX_PES) {
        for (int i = l; i < nc; i += 64) {
            const double li = clo[i], hi_ = chi[i];
            int cf = 0;
            for (int q = 0; q < nc; q++) cf |= (q != i) & (clo[q] <= hi_) & (li <= chi[q]);
            if (cf) ci[i] = -1 - ci[i];
            any |= cf;
        }
        any = __ballot(any) != 0ull;
        zz_wave_sync_lds();
    }
    if (any) {
        const float *xn = a.xn + (size_t)s * a.D;
        for (int i = 0; i < nc; i++) {                         // wave-uniform
            const int ce = ci[i];
            if (ce >= 0) continue;
            const int e = -1 - ce;
            const float v = zz_gemma_chain(a.router + (size_t)e * a.D, xn, a.D, a.bias, e);
            zz_wave_sync_lds();
            if (l == 0) {
                clo[i] = chi[i] = (double)v;
                ci[i] = e;
            }
            zz_wave_sync_lds();
        }
        if (l == 0 && write) atomicAdd(a.diag + 2, 1u);
    }

    // 5. rank candidates by (centre desc, index asc); after step 4 two equal centres
    // are two equal exact values, whose order the lower index decides
    int tie = 0;
    for (int i = l; i < nc; i += 64) {
        const int e = ci[i];
        const double me = 0.5 * (clo[i] + chi[i]);
        int rk = 0, eq = 0;
        for (int q = 0; q < nc; q++) {
            const int f = ci[q];
            const double mf = 0.5 * (clo[q] + chi[q]);
            rk += (f != e) & ((mf > me) | ((mf == me) & (f < e)));
            eq |= (f != e) & (mf == me);
        }
        if (rk < K) {
            h.idx[rk] = e;
            h.topv[rk] = (float)me;
            tie |= eq;
        }
    }
    ties |= __ballot(tie) != 0ull;
    }                                                    // general passes
    zz_wave_sync_lds();

    if (gates) {
        // slot l's centre and scale from the lane that loaded them
        const int ej = l < K ? h.idx[l] : 0, own = ej & 63, jj = ej >> 6;
        double cj = 0.0;
        float pj = 1.0f;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            const double c = __shfl(cv[j], own, 64);
            const float q = __shfl(pv[j], own, 64);
            if (jj == j) {
                cj = c;
                pj = q;
            }
        }
        zz_topk_gates(a, s, h, cj, pj, write);
    }
    if (l == 0 && ties && write) atomicAdd(a.diag + 3, 1u);
}

// The gate weights of a selection that zz_topk_wave(..., gates = false) left in lds:
// each slot's centre and scale read again from memory.
__device__ __forceinline__ void zz_topk_wave_gates(const ZzTopkArgs &a, int s, char *lds, bool write) {
    ZzTopkWaveHdr &h = *(ZzTopkWaveHdr *)lds;
    const int l = threadIdx.x & 63;
    double cj = 0.0;
    float pj = 1.0f;
    if (l < a.K) {
        const int ej = h.idx[l];
        cj = a.cen[(size_t)s * a.E + ej];
        if (a.gating == ZZ_GATE_SOFTMAX_PES) pj = a.pes[ej];
    }
    zz_topk_gates(a, s, h, cj, pj, write);
}

// experts per lane of zz_topk_wave for E experts
__host__ __device__ inline int zz_topk_epl(int E) { return E <= 64 ? 1 : (E <= 128 ? 2 : (E <= 256 ? 4 : 8)); }

// zz_topk_wave with the lane count chosen at run time
__device__ __forceinline__ void zz_topk_wave_any(const ZzTopkArgs &a, int s, char *lds, bool write = true,
                                                 bool gates = true) {
    switch (zz_topk_epl(a.E)) {
    case 1: zz_topk_wave<1>(a, s, lds, write, gates); break;
    case 2: zz_topk_wave<2>(a, s, lds, write, gates); break;
    case 4: zz_topk_wave<4>(a, s, lds, write, gates); break;
    default: zz_topk_wave<8>(a, s, lds, write, gates); break;
    }
}
