// zz_api.hip -- host side of libzzmoe.so: the gpu.h-compatible entry points
// (include/zz_gpu.h) and the MoE-layer entry points (include/zz_moe.h).
//
// State is process-global and single-caller, as the reference backend's is
// (metal.mm:289-296): one device, one library stream at default priority, a
// registry of uploaded host ranges, and the registered MoE layers with their
// HBM slot tables and per-layer workspaces.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_manifest.h"
#include "../../include/zz_moe.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

static char g_err[512];
void zz_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
#define ZZ_FAIL(...)               \
    do {                           \
        zz_set_error(__VA_ARGS__); \
        return 0;                  \
    } while (0)

static int g_ready = 0;
// batches of at most this many tokens take the three-launch decode path
// (ZZ_DECODE_MAX_S, 0 turns it off; never above ZZ_DEC_MAXS)
static int g_dec_max_s = ZZ_DEC_MAXS;
static int g_exact_min_s = 16;          // ZZ_EXACT_LOGITS_MIN_S
static char g_name[128] = "none";
static hipStream_t g_stream = nullptr;
static unsigned *g_diag = nullptr;          // device counters, see zz_moe_stats
static unsigned long long g_mem_gen = 1;    // see zz_lib_mem_gen

// Scratch of zz_moe_forward_dev_noalloc: the workspace of one chunk, in a
// file-scope device array that the code object brings with it (zero at load, held
// by each device until the process ends). In host code `scratch` names a host-side
// stand-in, not device memory: gpu_init takes the array's device address on each
// device once with hipGetSymbolAddress, and only that address is used.
#define ZZ_SCRATCH_BYTES ((size_t)64 << 20)
#define ZZ_MAX_DEVICES 16
static __device__ __align__(256) unsigned char scratch[ZZ_SCRATCH_BYTES];
static char *g_scratch[ZZ_MAX_DEVICES];     // scratch's address on device i
static hipError_t g_scratch_err = hipSuccess;

static ZzRanges g_maps;                      // gpu_map's host ranges (zz_manifest.h)

// ----------------------------------------------------------------- gpu.h ABI
extern "C" int gpu_init(void) {
    if (g_ready) return 1;
    const char *off = getenv("ZZ_DISABLE");
    if (off && off[0] == '1') ZZ_FAIL("disabled by ZZ_DISABLE");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) ZZ_FAIL("no HIP device");
    hipDeviceProp_t p;
    ZZ_CHECK(hipSetDevice(0));
    ZZ_CHECK(hipGetDeviceProperties(&p, 0));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) ZZ_FAIL("device %s is not gfx950", p.gcnArchName);
    snprintf(g_name, sizeof g_name, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    // the scratch array's address on this device (device 0, current since above);
    // without it only zz_moe_forward_dev_noalloc declines, with this error
    if (!g_scratch[0]) {
        void *sp = nullptr;
        g_scratch_err = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (g_scratch_err == hipSuccess && sp) g_scratch[0] = (char *)sp;
    }
    // the library's stream, what a NULL stream argument means: a blocking stream, so it
    // is ordered with the legacy default stream both ways, as a caller passing the
    // default stream's handle (0, e.g. torch's current stream) expects
    ZZ_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamDefault));
    ZZ_CHECK(hipMalloc(&g_diag, 16 * sizeof(unsigned)));
    ZZ_CHECK(hipMemset(g_diag, 0, 16 * sizeof(unsigned)));
    // batches from this size on take the exact serial router chains, smaller ones the
    // certified parallel logits with exact replay of contested chains
    const char *em = getenv("ZZ_EXACT_LOGITS_MIN_S");
    if (em) g_exact_min_s = atoi(em) < 1 ? 1 : atoi(em);
    const char *dm = getenv("ZZ_DECODE_MAX_S");
    if (dm) g_dec_max_s = atoi(dm) < 0 ? 0 : (atoi(dm) > ZZ_DEC_MAXS ? ZZ_DEC_MAXS : atoi(dm));
    g_ready = 1;
    return 1;
}

extern "C" int gpu_ready(void) { return g_ready; }
extern "C" const char *gpu_name(void) { return g_name; }


// A range inside an existing mapping is re-uploaded in place (the refresh an
// engine does after rewriting a mapped buffer). A range that only overlaps older
// mappings means that host memory was released and reused: those mappings are
// dropped so a lookup can never return bytes from the previous owner.
extern "C" int gpu_map(const void *p, size_t n) {
    if (!g_ready || !p || !n) ZZ_FAIL("gpu_map: not ready or empty range");
    if (ZzRange *m = g_maps.find(p, n)) {
        const size_t off = (uintptr_t)p - m->host;
        ZZ_CHECK(hipMemcpy(m->dev + off, p, n, hipMemcpyHostToDevice));
        zz_fp_take(*m, off, n);
        return 1;
    }
    g_maps.drop_overlaps(p, n, [](const ZzRange &m) { (void)hipFree(m.dev); });
    uint8_t *dev = nullptr;
    ZZ_CHECK(hipMalloc(&dev, n));
    if (hipMemcpy(dev, p, n, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(dev);
        ZZ_FAIL("gpu_map: upload failed");
    }
    zz_fp_take(g_maps.add(p, n, dev), 0, n);
    return 1;
}

// tensors gpu_matmul found rewritten on the host since their last upload
static long long g_map_refreshes = 0;
extern "C" long long zz_gpu_map_refreshes(void) { return g_map_refreshes; }

static int64_t fmt_tensor_bytes(int fmt, int O, int I) {
    if (fmt == ZZ_FMT_Q40) return (int64_t)O * (I / ZZ_BLK) * 18;
    if (fmt == ZZ_FMT_Q80) return (int64_t)O * (I / ZZ_BLK) * 34;
    if (fmt == ZZ_FMT_TQ2) return (int64_t)O * 4 + (int64_t)O * (I / 4);
    if (fmt == ZZ_FMT_Q4A) return (int64_t)O * (I / 64) * 36;        // tq2.h:287-292
    return -1;
}

// scratch for the matmul path, grown on demand
static float *g_mx = nullptr, *g_my = nullptr;
static size_t g_mxn = 0, g_myn = 0;

static int grow(float **p, size_t *cap, size_t n) {
    if (n <= *cap) return 1;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    ZZ_CHECK(hipMalloc(p, n * sizeof(float)));
    *cap = n;
    return 1;
}

extern "C" int gpu_matmul(int fmt, float *y, const uint8_t *W, const float *x, int O, int I, int S) {
    if (!g_ready) ZZ_FAIL("gpu_matmul: not ready");
    if (fmt != ZZ_FMT_Q40 && fmt != ZZ_FMT_Q80 && fmt != ZZ_FMT_TQ2 && fmt != ZZ_FMT_Q4A)
        ZZ_FAIL("gpu_matmul: fmt %d declined", fmt);
    const int grp = fmt == ZZ_FMT_TQ2 || fmt == ZZ_FMT_Q4A ? 64 : 32;
    if (O <= 0 || I <= 0 || S <= 0 || I % grp) ZZ_FAIL("gpu_matmul: bad shape");
    const size_t wb = (size_t)fmt_tensor_bytes(fmt, O, I);
    ZzRange *m = g_maps.find(W, wb);
    if (!m) ZZ_FAIL("gpu_matmul: W not inside a gpu_map'd range");
    const size_t off = (uintptr_t)W - m->host;
    if (zz_fp_changed(*m, off, wb)) {            // refilled since its upload: refresh it
        ZZ_CHECK(hipMemcpy(m->dev + off, W, wb, hipMemcpyHostToDevice));
        zz_fp_take(*m, off, wb);
        g_map_refreshes++;
    }
    const uint8_t *dW = m->dev + off;
    if (!grow(&g_mx, &g_mxn, (size_t)S * I) || !grow(&g_my, &g_myn, (size_t)S * O)) return 0;
    ZZ_CHECK(hipMemcpyAsync(g_mx, x, sizeof(float) * (size_t)S * I, hipMemcpyHostToDevice, g_stream));
    if (!zz_launch_matmul_f32(fmt, g_my, dW, g_mx, O, I, S, g_stream)) ZZ_FAIL("gpu_matmul: launch failed");
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    ZZ_CHECK(hipMemcpy(y, g_my, sizeof(float) * (size_t)S * O, hipMemcpyDeviceToHost));
    return 1;
}

extern "C" int gpu_q40_matmul(float *y, const uint8_t *W, const float *x, int O, int I, int S) {
    return gpu_matmul(ZZ_FMT_Q40, y, W, x, O, I, S);
}

// ----------------------------------------------------------------- MoE layers
struct Workspace {
    int S = 0;                  // tokens per chunk this workspace holds
    float *in = nullptr, *out = nullptr, *xn = nullptr;
    int8_t *xq = nullptr;
    float *xs = nullptr, *xt = nullptr;
    int *xsum = nullptr;
    double *cen = nullptr, *bnd = nullptr;
    int *eidx = nullptr;
    float *ewt = nullptr, *topv = nullptr;
    int *ptok = nullptr, *pslot = nullptr, *ppos = nullptr;
    float *pwt = nullptr;
    int *uniq = nullptr, *uoff = nullptr, *ucnt = nullptr, *meta = nullptr;
    ZzItem *items = nullptr;
    int8_t *hq = nullptr;
    float *hs = nullptr;
    int *hsum = nullptr;
    float *y = nullptr;
    double *ss = nullptr;       // decode post-norm per-tile sums of squares
    void *block = nullptr;      // one allocation holds everything above
};

struct Layer {
    zz_moe_desc d;
    ZzLayout lay;
    int64_t rec_bytes, src_gate, src_up, src_down;
    float *router = nullptr, *rscale = nullptr, *pes = nullptr, *bias = nullptr;
    float *pre_ln = nullptr, *post_ln = nullptr;
    uint8_t *slots = nullptr;   // E * lay.bytes: the HBM slot table
    uint8_t *staging = nullptr; // one reference record, for uploads
    std::vector<char> present;
    int n_present = 0;
    Workspace ws;
    int last_S = 0;             // tokens of the last chunk of the last forward
    bool last_dec = false;      // whether that chunk ran the decode kernels (hidden by flat pair)
    int pending_S = -1;         // begin/end state
};
static std::vector<Layer *> g_layers;

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

ZzTensor zz_make_tensor(int fmt, int O, int I, int64_t *cursor) {
    ZzTensor t;
    t.fmt = fmt;
    t.O = O;
    t.I = I;
    if (fmt == ZZ_FMT_TQ2) {
        t.off_s = *cursor;
        *cursor = align256(*cursor + (int64_t)O * 4);
        t.off_q = *cursor;
        *cursor = align256(*cursor + (int64_t)O * (I / 4));
    } else {
        t.off_q = *cursor;
        *cursor = align256(*cursor + (int64_t)O * (I / ZZ_BLK) * zz_pbytes(t));
        t.off_s = *cursor;
        *cursor = align256(*cursor + (int64_t)O * (I / ZZ_BLK) * 2);
    }
    return t;
}

static int desc_ok(const zz_moe_desc *d) {
    if (!d) return 0;
    if (d->D <= 0 || d->MI <= 0 || d->D % 64 || d->MI % 64 || d->D > ZZ_MAXD || d->MI > ZZ_MAXD) return 0;
    if (d->E <= 0 || d->E > ZZ_MAXE || d->K < 1 || d->K > ZZ_MAXK || d->K > d->E) return 0;
    if (d->gating < 0 || d->gating > 4 || d->act < 0 || d->act > 2) return 0;
    if (d->gating == ZZ_GATE_DENSE && (d->E != 1 || d->K != 1 || d->use_bias)) return 0;
    if (d->gating == ZZ_GATE_GROUPED &&                 // ling.c:352-353
        (d->n_group < 1 || d->n_group > ZZ_MAXGROUP || d->E % d->n_group || d->topk_group < 1 ||
         d->topk_group > d->n_group || d->K > d->topk_group * (d->E / d->n_group)))
        return 0;
    int f[3] = {d->fmt_gate, d->fmt_up, d->fmt_down};
    for (int i = 0; i < 3; i++)
        if (f[i] != ZZ_FMT_Q40 && f[i] != ZZ_FMT_Q80 && f[i] != ZZ_FMT_TQ2) return 0;
    // the tq2 -1 offset is settled once per activation (tq2.h:29-37): gate and up
    // share the input, so either both or neither of them is ternary
    if ((d->fmt_gate == ZZ_FMT_TQ2) != (d->fmt_up == ZZ_FMT_TQ2)) return 0;
    return 1;
}

extern "C" int64_t zz_moe_record_bytes(const zz_moe_desc *d) {
    if (!desc_ok(d)) return -1;
    return fmt_tensor_bytes(d->fmt_gate, d->MI, d->D) + fmt_tensor_bytes(d->fmt_up, d->MI, d->D) +
           fmt_tensor_bytes(d->fmt_down, d->D, d->MI);
}

static int upload_f32(float **dst, const float *src, size_t n) {
    if (!src) return 1;
    ZZ_CHECK(hipMalloc(dst, n * sizeof(float)));
    ZZ_CHECK(hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice));
    return 1;
}

static void free_layer(Layer *L) {
    if (!L) return;
    zz_lib_mem_bump();
    void *ps[] = {L->router, L->rscale, L->pes, L->bias, L->pre_ln, L->post_ln, L->slots,
                  L->staging, L->ws.block};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    delete L;
}

extern "C" int zz_moe_layer_create(const zz_moe_desc *d, const zz_moe_weights *w) {
    if (!g_ready) { zz_set_error("zz_moe_layer_create: gpu_init first"); return -1; }
    const bool dense = desc_ok(d) && d->gating == ZZ_GATE_DENSE;
    if (!desc_ok(d) || !w || (!dense && !w->router)) { zz_set_error("zz_moe_layer_create: bad descriptor"); return -1; }
    if (d->gating == ZZ_GATE_SOFTMAX_PES && (!w->router_scale || !w->pes || !w->pre_ln || !w->post_ln)) {
        zz_set_error("zz_moe_layer_create: gemma gating needs scale, pes and both norms");
        return -1;
    }
    if (dense && (!w->pre_ln || !w->post_ln)) {
        zz_set_error("zz_moe_layer_create: the dense branch needs both norms");
        return -1;
    }
    const bool norms = d->gating == ZZ_GATE_SOFTMAX_PES || dense;
    if (d->use_bias && !w->bias) { zz_set_error("zz_moe_layer_create: use_bias without bias"); return -1; }
    Layer *L = new Layer();
    L->d = *d;
    int64_t cur = 0;
    L->lay.gate = zz_make_tensor(d->fmt_gate, d->MI, d->D, &cur);
    L->lay.up = zz_make_tensor(d->fmt_up, d->MI, d->D, &cur);
    L->lay.down = zz_make_tensor(d->fmt_down, d->D, d->MI, &cur);
    L->lay.bytes = cur;
    L->src_gate = 0;
    L->src_up = fmt_tensor_bytes(d->fmt_gate, d->MI, d->D);
    L->src_down = L->src_up + fmt_tensor_bytes(d->fmt_up, d->MI, d->D);
    L->rec_bytes = L->src_down + fmt_tensor_bytes(d->fmt_down, d->D, d->MI);
    bool ok = upload_f32(&L->router, dense ? nullptr : w->router, (size_t)d->E * d->D) &&
              upload_f32(&L->rscale, d->gating == ZZ_GATE_SOFTMAX_PES ? w->router_scale : nullptr, d->D) &&
              upload_f32(&L->pes, d->gating == ZZ_GATE_SOFTMAX_PES ? w->pes : nullptr, d->E) &&
              upload_f32(&L->bias, d->use_bias ? w->bias : nullptr, d->E) &&
              upload_f32(&L->pre_ln, norms ? w->pre_ln : nullptr, d->D) &&
              upload_f32(&L->post_ln, norms ? w->post_ln : nullptr, d->D) &&
              hipMalloc(&L->slots, (size_t)d->E * L->lay.bytes) == hipSuccess &&
              hipMalloc(&L->staging, (size_t)L->rec_bytes) == hipSuccess;
    if (!ok) {
        zz_set_error("zz_moe_layer_create: device allocation failed");
        free_layer(L);
        return -1;
    }
    L->present.assign(d->E, 0);
    for (size_t i = 0; i < g_layers.size(); i++)
        if (!g_layers[i]) { g_layers[i] = L; return (int)i; }
    g_layers.push_back(L);
    return (int)g_layers.size() - 1;
}

static Layer *get_layer(int id) {
    if (!g_ready || id < 0 || id >= (int)g_layers.size()) return nullptr;
    return g_layers[id];
}

// library internals shared with zz_gemma.hip
hipStream_t zz_lib_stream() { return g_stream; }
int zz_lib_ready() { return g_ready; }
unsigned long long zz_lib_mem_gen() { return g_mem_gen; }
void zz_lib_mem_bump() { g_mem_gen++; }
unsigned *zz_lib_diag() { return g_diag; }
const zz_moe_desc *zz_layer_desc(int id) {
    const Layer *L = get_layer(id);
    return L ? &L->d : nullptr;
}

extern "C" void zz_moe_layer_destroy(int id) {
    Layer *L = get_layer(id);
    if (!L) return;
    (void)hipStreamSynchronize(g_stream);
    free_layer(L);
    g_layers[id] = nullptr;
}

static int upload_common(Layer *L, int eid, const void *src, size_t n, hipMemcpyKind kind) {
    if (eid < 0 || eid >= L->d.E) ZZ_FAIL("upload: expert %d out of range", eid);
    if ((int64_t)n != L->rec_bytes) ZZ_FAIL("upload: record is %zu bytes, expected %lld", n, (long long)L->rec_bytes);
    ZZ_CHECK(hipMemcpyAsync(L->staging, src, n, kind, g_stream));
    ZzRepackArgs a;
    a.src = L->staging;
    a.src_gate = L->src_gate;
    a.src_up = L->src_up;
    a.src_down = L->src_down;
    a.dst = L->slots + (size_t)eid * L->lay.bytes;
    a.lay = L->lay;
    if (!zz_launch_repack(a, g_stream)) ZZ_FAIL("upload: repack launch failed");
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    if (!L->present[eid]) { L->present[eid] = 1; L->n_present++; }
    return 1;
}

extern "C" int zz_moe_expert_upload(int id, int eid, const uint8_t *rec, size_t n) {
    Layer *L = get_layer(id);
    if (!L || !rec) ZZ_FAIL("zz_moe_expert_upload: bad layer or record");
    return upload_common(L, eid, rec, n, hipMemcpyHostToDevice);
}

extern "C" int zz_moe_expert_upload_dev(int id, int eid, const void *d_rec, size_t n) {
    Layer *L = get_layer(id);
    if (!L || !d_rec) ZZ_FAIL("zz_moe_expert_upload_dev: bad layer or record");
    return upload_common(L, eid, d_rec, n, hipMemcpyDeviceToDevice);
}

// largest chunk one dispatch workgroup handles: S*K <= 8192 pairs and the two
// per-expert token bitmasks (2 * E * ceil(S/32) words) within 48 KB of LDS
static int chunk_tokens(const zz_moe_desc &d) {
    int by_pairs = 8192 / d.K;
    int by_masks = 32 * (6144 / d.E);
    return by_pairs < by_masks ? by_pairs : by_masks;
}

// Rows of the FFN work-item grid (slots per XCD): enough for the items of S tokens
// in chunks of <= tch (one expert's items may all sit on one XCD), so that the XCD
// placement of the dispatch kernel always fits.
static int zz_item_slots(int E, int P, int S, int tch) {
    const int items = (P < E ? P : E) + (P + tch - 1) / tch;
    return (items + 7) / 8 + (S + tch - 1) / tch;
}

// An expert's gate + up weight stream expressed in token columns of the FFN's
// epilogue work (the dispatch kernel's XCD balance): ~29 for q4_0, where 2.2 MB of
// weights take as long at HBM speed as 29 columns of 3 VALU operations per weight
// row and 32-weight block take on the XCD's SIMDs.
static int zz_weight_cost(const ZzLayout &lay, const zz_moe_desc &d) {
    const double bytes = (double)(lay.gate.fmt == ZZ_FMT_Q80 ? 34 : lay.gate.fmt == ZZ_FMT_TQ2 ? 8.125 : 18) / 32.0 +
                         (double)(lay.up.fmt == ZZ_FMT_Q80 ? 34 : lay.up.fmt == ZZ_FMT_TQ2 ? 8.125 : 18) / 32.0;
    const int c = (int)(29.0 * bytes / 1.125 + 0.5);
    return c < 1 ? 1 : c;
}

// Lays the workspace of S tokens of layer d out from `base` (nullptr: only
// measures). host_io adds the in/out staging rows that only the host-pointer
// forms use. Returns the bytes the layout spans.
static size_t ws_layout(const zz_moe_desc &d, int S, bool host_io, char *base, Workspace *w) {
    const size_t P = (size_t)S * d.K, nbD = d.D / ZZ_BLK, nbM = d.MI / ZZ_BLK;
    // FFN work-item slots: 8 per row of the XCD-placed item grid (zz_item_slots)
    const size_t nitems = 8 * (size_t)zz_item_slots(d.E, (int)P, S, 4) + 8;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t o = off;
        off = (off + bytes + 255) & ~(size_t)255;
        return base ? base + o : nullptr;
    };
    Workspace v;
    v.S = S;
    v.in = (float *)take(host_io ? 4 * S * (size_t)d.D : 0);
    v.out = (float *)take(host_io ? 4 * S * (size_t)d.D : 0);
    v.xn = (float *)take(4 * S * (size_t)d.D);
    v.xq = (int8_t *)take(S * (size_t)d.D); v.xs = (float *)take(4 * S * nbD); v.xsum = (int *)take(4 * S * nbD);
    v.xt = (float *)take(4 * (size_t)S);
    v.cen = (double *)take(8 * S * (size_t)d.E); v.bnd = (double *)take(8 * S * (size_t)d.E);
    v.eidx = (int *)take(4 * P); v.ewt = (float *)take(4 * P); v.topv = (float *)take(4 * P);
    v.ptok = (int *)take(4 * P); v.pslot = (int *)take(4 * P); v.ppos = (int *)take(4 * P); v.pwt = (float *)take(4 * P);
    v.uniq = (int *)take(4 * (size_t)d.E); v.uoff = (int *)take(4 * (size_t)d.E); v.ucnt = (int *)take(4 * (size_t)d.E);
    v.meta = (int *)take(64); v.items = (ZzItem *)take(sizeof(ZzItem) * nitems);
    v.hq = (int8_t *)take(P * d.MI); v.hs = (float *)take(4 * P * nbM); v.hsum = (int *)take(4 * P * nbM);
    v.y = (float *)take(4 * P * d.D); v.ss = (double *)take(8 * S * (size_t)(d.D / 16));
    if (!host_io) v.in = v.out = nullptr;
    if (w) *w = v;
    return off;
}

static int ensure_ws(Layer *L, int S) {
    Workspace &w = L->ws;
    if (S <= w.S) return 1;
    const size_t bytes = ws_layout(L->d, S, true, nullptr, nullptr);
    void *blk = nullptr;
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    ZZ_CHECK(hipMalloc(&blk, bytes));
    if (w.block) (void)hipFree(w.block);
    zz_lib_mem_bump();
    ws_layout(L->d, S, true, (char *)blk, &w);
    w.block = blk;
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    return 1;
}

// ----------------------------------------------------------------- profiling
struct ProfRec {
    int k;
    hipEvent_t a, b;
};
static int g_prof = 0;
static std::vector<ProfRec> g_prof_recs;
static std::vector<hipEvent_t> g_event_pool;

static hipEvent_t prof_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

struct ProfScope {             // brackets one kernel launch with two events
    int k;
    hipStream_t st;
    hipEvent_t a = nullptr;
    ProfScope(int k_, hipStream_t st_) : k(k_), st(st_) {
        if (g_prof) {
            a = prof_event();
            (void)hipEventRecord(a, st);
        }
    }
    ~ProfScope() {
        if (g_prof && a) {
            hipEvent_t b = prof_event();
            (void)hipEventRecord(b, st);
            g_prof_recs.push_back({k, a, b});
        }
    }
};

// internal: event timing off while a HIP graph is captured; returns the old state
int zz_lib_prof_set(int on) {
    const int was = g_prof;
    g_prof = on;
    return was;
}

extern "C" int zz_moe_profile(int on) {
    if (!g_ready) ZZ_FAIL("zz_moe_profile: not ready");
    (void)hipDeviceSynchronize();
    // switching off keeps the records (and their events) for zz_moe_profile_read;
    // only a new session recycles them, so no event is ever in the pool and in a
    // record at once
    if (on) {
        for (ProfRec &r : g_prof_recs) { g_event_pool.push_back(r.a); g_event_pool.push_back(r.b); }
        g_prof_recs.clear();
    }
    g_prof = on;
    return 1;
}

extern "C" int zz_moe_profile_read(double *ms, int *launches, int n) {
    if (!g_ready || !ms || !launches) ZZ_FAIL("zz_moe_profile_read: bad arguments");
    ZZ_CHECK(hipDeviceSynchronize());
    for (int k = 0; k < n; k++) { ms[k] = 0.0; launches[k] = 0; }
    for (ProfRec &r : g_prof_recs) {
        float t = 0.0f;
        ZZ_CHECK(hipEventElapsedTime(&t, r.a, r.b));
        if (r.k < n) { ms[r.k] += t; launches[r.k]++; }
    }
    return ZZ_K_COUNT;
}

// One chunk of S <= chunk_tokens tokens: in/out device pointers.
// decode-sized batches whose hidden rows fit the decode kernels' LDS take the GEMV
// path; larger ones the matrix cores
// The decode kernels read each (token, slot) pair's expert rows, the matrix-core path
// each distinct expert's once: measured on the MI355X (bench.py layers), decode wins
// for q4_0 / q8_0 experts up to S = 2 (gemma S=2: 45.9 us against 55.1; S=3: 62.9
// against 60.0; lfm S=4: 62.1 against 53.7) and for tq2's quarter-size rows up to S = 4
// (maple S=4: 51.5 against 58.7).
static bool takes_decode(const zz_moe_desc &d, int S) {
    const int lim = d.fmt_gate == ZZ_FMT_TQ2 ? ZZ_DEC_MAXS : 2;
    return S <= g_dec_max_s && S <= lim && zz_dec_fits(S, d.K, d.MI);
}

// Kernel arguments of one chunk of S <= chunk_tokens rows of layer L.
struct ChunkArgs {
    ZzPrepArgs pa;
    ZzLogitArgs la;
    ZzTopkArgs ta;
    ZzDispatchArgs da;
    ZzFfnArgs fa;
    bool dense, gemma, dec;
    int P, max_items;
};

// zz_moe_dots: while it runs, the FFN kernels also store their per-block int32 dots
static int32_t *g_dbg_up = nullptr, *g_dbg_dn = nullptr;

static ChunkArgs chunk_args(Layer *L, Workspace &w, const float *d_in, int S) {
    const zz_moe_desc &d = L->d;
    ChunkArgs c;
    memset(&c, 0, sizeof c);
    c.dense = d.gating == ZZ_GATE_DENSE;            // gemma's norms, no router
    c.gemma = d.gating == ZZ_GATE_SOFTMAX_PES || c.dense;
    const bool tq_in = d.fmt_gate == ZZ_FMT_TQ2;
    c.P = S * d.K;

    ZzPrepArgs &pa = c.pa;
    pa.D = d.D; pa.gemma = c.gemma; pa.eps = d.eps; pa.in = d_in;
    pa.router_scale = L->rscale; pa.pre_ln = L->pre_ln; pa.xn = w.xn;
    pa.xq = w.xq; pa.xs = w.xs; pa.xsum = w.xsum; pa.xt = tq_in ? w.xt : nullptr; pa.diag = g_diag;
    pa.route_eidx = c.dense ? w.eidx : nullptr; pa.route_ewt = c.dense ? w.ewt : nullptr;

    ZzLogitArgs &la = c.la;
    la.D = d.D; la.E = d.E; la.gating = d.gating; la.S = S; la.router = L->router; la.xn = w.xn; la.x = d_in;
    la.bias = c.gemma && d.use_bias ? L->bias : nullptr; la.cen = w.cen; la.bnd = w.bnd; la.diag = g_diag;
    la.exact_min_s = g_exact_min_s;

    ZzTopkArgs &ta = c.ta;
    ta.D = d.D; ta.E = d.E; ta.K = d.K; ta.gating = d.gating; ta.norm_topk = d.norm_topk;
    ta.n_group = d.n_group; ta.topk_group = d.topk_group;
    ta.routed_scaling = d.routed_scaling; ta.cen = w.cen; ta.bnd = w.bnd; ta.router = L->router;
    ta.xn = w.xn; ta.bias = d.use_bias ? L->bias : nullptr; ta.pes = L->pes; ta.eidx = w.eidx;
    ta.ewt = w.ewt; ta.topv = w.topv; ta.diag = g_diag;

    // decode-sized batches take the GEMV path; larger ones the matrix cores, on
    // work items of up to ZZ_MMA_TOKENS tokens of one expert
    c.dec = takes_decode(d, S);
    const int tch = c.dec ? ZZ_DEC_MAXS : ZZ_MMA_TOKENS;
    ZzDispatchArgs &da = c.da;
    da.P = c.P; da.E = d.E; da.K = d.K; da.tch = tch; da.eidx = w.eidx; da.ewt = w.ewt;
    da.xslots = zz_item_slots(d.E, c.P, S, tch);
    da.wcost = zz_weight_cost(L->lay, d);
    da.ptok = w.ptok; da.pslot = w.pslot; da.pwt = w.pwt; da.ppos = w.ppos; da.uniq = w.uniq;
    da.uoff = w.uoff; da.ucnt = w.ucnt; da.items = w.items; da.meta = w.meta;

    ZzFfnArgs &fa = c.fa;
    fa.D = d.D; fa.MI = d.MI; fa.K = d.K; fa.act = d.act; fa.clamp = d.clamp;
    fa.experts = L->slots; fa.estride = L->lay.bytes; fa.lay = L->lay; fa.items = w.items;
    fa.meta = w.meta; fa.ptok = w.ptok; fa.xq = w.xq; fa.xs = w.xs; fa.xsum = w.xsum; fa.xt = w.xt;
    fa.hq = w.hq; fa.hs = w.hs; fa.hsum = w.hsum; fa.y = w.y;
    fa.pslot = w.pslot; fa.dbg_up = g_dbg_up; fa.dbg_dn = g_dbg_dn;
    c.max_items = 8 * da.xslots;
    return c;
}

static int run_chunk(Layer *L, Workspace &w, const float *d_in, float *d_out, int S, hipStream_t st) {
    const zz_moe_desc &d = L->d;
    ChunkArgs c = chunk_args(L, w, d_in, S);

    if (c.dec) {
        ZzDecRouteArgs ra;
        memset(&ra, 0, sizeof ra);
        ra.prep = c.pa; ra.lg = c.la; ra.tk = c.ta; ra.dp = c.da; ra.S = S; ra.dense = c.dense;
        if (!(ProfScope(ZZ_K_DEC_ROUTE, st), zz_launch_dec_logits(ra, st))) ZZ_FAIL("decode router launch failed");
        ZzDecUpArgs ua;
        memset(&ua, 0, sizeof ua);
        ua.f = c.fa; ua.tk = c.ta; ua.dense = c.dense; ua.pk = c.P;
        ZzDecDownArgs dd;
        memset(&dd, 0, sizeof dd);
        dd.f = c.fa; dd.S = S; dd.K = d.K; dd.E = d.E; dd.eidx = w.eidx; dd.ewt = w.ewt;
        dd.out = d_out; dd.ss = c.gemma ? w.ss : nullptr;
        if (!(ProfScope(ZZ_K_FFN_UP, st), zz_launch_dec_up(ua, S, st))) ZZ_FAIL("ffn_up launch failed");
        if (!(ProfScope(ZZ_K_DEC_DOWN, st), zz_launch_dec_down(dd, st))) ZZ_FAIL("decode down launch failed");
        if (c.gemma && !(ProfScope(ZZ_K_COMBINE, st), zz_launch_dec_norm(d_out, L->post_ln, w.ss, d.D, d.eps, S, st)))
            ZZ_FAIL("decode post-norm launch failed");
        if (&w == &L->ws) {                      // what zz_moe_debug dumps
            L->last_S = S;
            L->last_dec = true;
        }
        return 1;
    }
    if (!(ProfScope(ZZ_K_PREP, st), zz_launch_prep(c.pa, S, st))) ZZ_FAIL("prep launch failed");
    if (!c.dense && !(ProfScope(ZZ_K_LOGITS, st), zz_launch_logits(c.la, S, st))) ZZ_FAIL("logits launch failed");
    if (!c.dense && !(ProfScope(ZZ_K_TOPK, st), zz_launch_topk(c.ta, S, st))) ZZ_FAIL("topk launch failed");
    if (!(ProfScope(ZZ_K_DISPATCH, st), zz_launch_dispatch(c.da, st))) ZZ_FAIL("dispatch launch failed");
    if (!(ProfScope(ZZ_K_FFN_UP, st), zz_launch_up_mfma(c.fa, c.max_items, st))) ZZ_FAIL("ffn_up launch failed");
    if (!(ProfScope(ZZ_K_FFN_DOWN, st), zz_launch_down_mfma(c.fa, c.max_items, st))) ZZ_FAIL("ffn_down launch failed");

    ZzCombineArgs ca;
    ca.D = d.D; ca.K = d.K; ca.gemma = c.gemma; ca.eps = d.eps; ca.y = w.y;
    ca.ewt = w.ewt; ca.post_ln = L->post_ln; ca.out = d_out;
    if (!(ProfScope(ZZ_K_COMBINE, st), zz_launch_combine(ca, S, st))) ZZ_FAIL("combine launch failed");
    if (&w == &L->ws) {
        L->last_S = S;
        L->last_dec = false;
    }
    return 1;
}

// The decode rows of a gemma FFN block (zz_gemma.hip) with the dense layer fused into
// the routed layer's four launches: the router kernel also quantises the dense
// branch's input, the gate/up kernel runs its rows as extra grid rows, the down
// kernel its output rows beside the routed pairs', and one final kernel applies
// both post-norms and the layer combine. H is updated in place; h1/h2 [S, D] hold
// the dense and routed outputs before their norms. Returns 1 when done, 0 on a
// failure, -1 when the layers or S do not take this path.
int zz_block_decode_fits(int moe_id, int dense_id, int S) {
    Layer *L = get_layer(moe_id), *N = get_layer(dense_id);
    if (!L || !N || S <= 0) return 0;
    const zz_moe_desc &d = L->d, &dn = N->d;
    // the fused block rows keep the decode kernels up to ZZ_DEC_MAXS: they also save
    // the dense branch its own launches and stream
    return !(d.gating != ZZ_GATE_SOFTMAX_PES || dn.gating != ZZ_GATE_DENSE || d.D != dn.D || S > g_dec_max_s ||
             !zz_dec_fits(S, d.K, d.MI) || S > chunk_tokens(d) || d.fmt_down != dn.fmt_down ||
             d.fmt_down == ZZ_FMT_TQ2 || dn.fmt_gate == ZZ_FMT_TQ2 || dn.fmt_up == ZZ_FMT_TQ2 ||
             d.fmt_gate == ZZ_FMT_TQ2 || !zz_dec_fits2(S, d.K, d.MI, dn.MI));
}

int zz_block_decode(int moe_id, int dense_id, float *d_H, float *d_h1, float *d_h2, const float *post_ln,
                    float ls, int S, int *d_eidx, float *d_ewt, hipStream_t st, const ZzDecFinalArgs *pend_in,
                    ZzDecFinalArgs *pend_out) {
    if (!zz_block_decode_fits(moe_id, dense_id, S)) return -1;
    Layer *L = get_layer(moe_id), *N = get_layer(dense_id);
    const zz_moe_desc &d = L->d, &dn = N->d;
    if (pend_in && (pend_in->Hout != d_H || pend_in->D != d.D || !zz_dec_fin_fits(S, d.D)))
        ZZ_FAIL("block: the deferred combine does not fit this block");
    if (L->n_present != d.E || N->n_present != dn.E) ZZ_FAIL("block: experts not uploaded");
    if (!ensure_ws(L, S) || !ensure_ws(N, S)) return 0;
    Workspace &w = L->ws, &wn = N->ws;
    ChunkArgs c = chunk_args(L, w, d_H, S), cn = chunk_args(N, wn, d_H, S);

    ZzDecRouteArgs ra;
    memset(&ra, 0, sizeof ra);
    ra.prep = c.pa; ra.lg = c.la; ra.tk = c.ta; ra.dp = c.da; ra.S = S; ra.dual = 1; ra.prep2 = cn.pa;
    if (pend_in) {
        ra.fin = 1;
        ra.fa = *pend_in;
    }
    if (!(ProfScope(ZZ_K_DEC_ROUTE, st), zz_launch_dec_logits(ra, st))) ZZ_FAIL("block: router launch failed");
    ZzDecUpArgs ua;
    memset(&ua, 0, sizeof ua);
    ua.f = c.fa; ua.tk = c.ta; ua.pk = c.P; ua.nd = S; ua.fd = cn.fa;
    if (!(ProfScope(ZZ_K_FFN_UP, st), zz_launch_dec_up(ua, S, st))) ZZ_FAIL("block: gate/up launch failed");
    ZzDecDownArgs dd;
    memset(&dd, 0, sizeof dd);
    dd.f = c.fa; dd.S = S; dd.K = d.K; dd.E = d.E; dd.eidx = w.eidx; dd.ewt = w.ewt;
    dd.out = d_h2; dd.ss = w.ss; dd.nd = S; dd.fd = cn.fa; dd.yd = d_h1; dd.ssd = wn.ss;
    if (!(ProfScope(ZZ_K_DEC_DOWN, st), zz_launch_dec_down(dd, st))) ZZ_FAIL("block: down launch failed");
    ZzDecFinalArgs fa;
    fa.D = d.D; fa.G = d.D / 16; fa.eps = d.eps; fa.ls = ls; fa.out = d_h2; fa.ss = w.ss; fa.post2 = L->post_ln;
    fa.yd = d_h1; fa.ssd = wn.ss; fa.post1 = N->post_ln; fa.post = post_ln; fa.H = d_H; fa.Hout = d_H;
    if (pend_out) {
        *pend_out = fa;
        pend_out->Hout = nullptr;
    } else if (!(ProfScope(ZZ_K_COMBINE, st), zz_launch_dec_final(fa, S, st))) {
        ZZ_FAIL("block: final launch failed");
    }
    if (d_eidx) ZZ_CHECK(hipMemcpyAsync(d_eidx, w.eidx, sizeof(int) * S * d.K, hipMemcpyDeviceToDevice, st));
    if (d_ewt) ZZ_CHECK(hipMemcpyAsync(d_ewt, w.ewt, sizeof(float) * S * d.K, hipMemcpyDeviceToDevice, st));
    L->last_S = N->last_S = S;                  // both layers' hidden rows by flat pair
    L->last_dec = N->last_dec = true;
    return 1;
}

// the chunks of a device-pointer forward, on workspace w (chunks of <= CH tokens)
static int run_chunks(Layer *L, Workspace &w, int CH, const float *d_in, float *d_out, int S, int *d_eidx,
                      float *d_ewt, hipStream_t st) {
    const zz_moe_desc &d = L->d;
    for (int s0 = 0; s0 < S; s0 += CH) {
        int n = S - s0 < CH ? S - s0 : CH;
        if (!run_chunk(L, w, d_in + (size_t)s0 * d.D, d_out + (size_t)s0 * d.D, n, st)) return 0;
        if (d_eidx) ZZ_CHECK(hipMemcpyAsync(d_eidx + (size_t)s0 * d.K, w.eidx, sizeof(int) * n * d.K, hipMemcpyDeviceToDevice, st));
        if (d_ewt) ZZ_CHECK(hipMemcpyAsync(d_ewt + (size_t)s0 * d.K, w.ewt, sizeof(float) * n * d.K, hipMemcpyDeviceToDevice, st));
    }
    return 1;
}

static int forward_dev(Layer *L, const float *d_in, float *d_out, int S, int *d_eidx, float *d_ewt,
                       hipStream_t st) {
    const zz_moe_desc &d = L->d;
    if (S <= 0) ZZ_FAIL("forward: S must be positive");
    if (L->n_present != d.E) ZZ_FAIL("forward: %d of %d experts uploaded", L->n_present, d.E);
    const int CH = chunk_tokens(d);
    if (!ensure_ws(L, S < CH ? S : CH)) return 0;
    if (!run_chunks(L, L->ws, CH, d_in, d_out, S, d_eidx, d_ewt, st)) return 0;
    return 1;
}

extern "C" int zz_moe_forward_dev(int id, const float *d_in, float *d_out, int S, int *d_eidx,
                                  float *d_ewt, void *stream) {
    Layer *L = get_layer(id);
    if (!L || !d_in || !d_out) ZZ_FAIL("zz_moe_forward_dev: bad arguments");
    return forward_dev(L, d_in, d_out, S, d_eidx, d_ewt, stream ? (hipStream_t)stream : g_stream);
}

// The device-pointer forward on the scratch array instead of the layer's workspace:
// no allocation at any point. Every call on a device shares its one array, which
// keeps the last call's contents; no kernel reads workspace memory it has not
// written in the same call, so nothing is cleared. Calls that overlap on one device
// (two streams, two threads) race on it.
extern "C" int zz_moe_forward_dev_noalloc(int id, const float *d_in, float *d_out, int S, int *d_eidx,
                                          float *d_ewt, void *stream) {
    Layer *L = get_layer(id);
    if (!L || !d_in || !d_out || S <= 0) ZZ_FAIL("zz_moe_forward_dev_noalloc: bad arguments");
    const zz_moe_desc &d = L->d;
    if (L->n_present != d.E) ZZ_FAIL("forward: %d of %d experts uploaded", L->n_present, d.E);
    int dev = -1;
    ZZ_CHECK(hipGetDevice(&dev));
    char *base = dev >= 0 && dev < ZZ_MAX_DEVICES ? g_scratch[dev] : nullptr;
    if (!base)
        ZZ_FAIL("zz_moe_forward_dev_noalloc: no scratch address on device %d (%s)", dev,
                hipGetErrorString(g_scratch_err));
    const int CH = chunk_tokens(d), S1 = S < CH ? S : CH;
    const size_t need = ws_layout(d, S1, false, nullptr, nullptr);
    if (need > ZZ_SCRATCH_BYTES)
        ZZ_FAIL("zz_moe_forward_dev_noalloc: %d tokens of this layer need %zu bytes of scratch, above its %zu: "
                "pass fewer tokens per call", S1, need, ZZ_SCRATCH_BYTES);
    Workspace w;
    ws_layout(d, S1, false, base, &w);
    const int prof = zz_lib_prof_set(0);           // its timing events would be created on demand
    const int ok = run_chunks(L, w, CH, d_in, d_out, S, d_eidx, d_ewt, stream ? (hipStream_t)stream : g_stream);
    zz_lib_prof_set(prof);
    return ok;
}

// Host-pointer forward: stage through the workspace chunk by chunk.
static int forward_host(Layer *L, const float *in, float *out, int S, int *eidx, float *ewt) {
    const zz_moe_desc &d = L->d;
    if (S <= 0 || !in || !out) ZZ_FAIL("forward: bad arguments");
    if (L->n_present != d.E) ZZ_FAIL("forward: %d of %d experts uploaded", L->n_present, d.E);
    const int CH = chunk_tokens(d);
    if (!ensure_ws(L, S < CH ? S : CH)) return 0;
    Workspace &w = L->ws;
    // results go to host staging first, so a failure leaves out/eidx/ewt untouched
    std::vector<float> o((size_t)S * d.D), wt((size_t)S * d.K);
    std::vector<int> ix((size_t)S * d.K);
    for (int s0 = 0; s0 < S; s0 += CH) {
        int n = S - s0 < CH ? S - s0 : CH;
        ZZ_CHECK(hipMemcpyAsync(w.in, in + (size_t)s0 * d.D, sizeof(float) * n * d.D, hipMemcpyHostToDevice, g_stream));
        if (!run_chunk(L, w, w.in, w.out, n, g_stream)) return 0;
        ZZ_CHECK(hipMemcpyAsync(o.data() + (size_t)s0 * d.D, w.out, sizeof(float) * n * d.D, hipMemcpyDeviceToHost, g_stream));
        ZZ_CHECK(hipMemcpyAsync(ix.data() + (size_t)s0 * d.K, w.eidx, sizeof(int) * n * d.K, hipMemcpyDeviceToHost, g_stream));
        ZZ_CHECK(hipMemcpyAsync(wt.data() + (size_t)s0 * d.K, w.ewt, sizeof(float) * n * d.K, hipMemcpyDeviceToHost, g_stream));
        ZZ_CHECK(hipStreamSynchronize(g_stream));
    }
    memcpy(out, o.data(), sizeof(float) * o.size());
    if (eidx) memcpy(eidx, ix.data(), sizeof(int) * ix.size());
    if (ewt) memcpy(ewt, wt.data(), sizeof(float) * wt.size());
    return 1;
}

extern "C" int zz_moe_forward(int id, const float *in, float *out, int S, int *eidx, float *ewt) {
    Layer *L = get_layer(id);
    if (!L) ZZ_FAIL("zz_moe_forward: no such layer");
    return forward_host(L, in, out, S, eidx, ewt);
}

// One synchronous forward on the FFN kernels' diagnostics builds, which also store
// every per-block int32 dot before its fp32 scaling. Unwritten entries keep the fill
// 0x80808080.
extern "C" int zz_moe_dots(int id, const float *in, int S, int32_t *up, int32_t *down) {
    Layer *L = get_layer(id);
    if (!L || !in || !up || !down || S <= 0) ZZ_FAIL("zz_moe_dots: bad arguments");
    const zz_moe_desc &d = L->d;
    if (S > chunk_tokens(d)) ZZ_FAIL("zz_moe_dots: S > %d", chunk_tokens(d));
    const size_t P = (size_t)S * d.K;
    const size_t nu = P * 2 * d.MI * (d.D / ZZ_BLK), nd = P * d.D * (d.MI / ZZ_BLK);
    if (nu + nd > ((size_t)64 << 20)) ZZ_FAIL("zz_moe_dots: %zu dots exceed the limit of 64 Mi", nu + nd);
    int32_t *du = nullptr, *dd = nullptr;
    ZZ_CHECK(hipMalloc(&du, 4 * nu));
    if (hipMalloc(&dd, 4 * nd) != hipSuccess) {
        (void)hipFree(du);
        ZZ_FAIL("zz_moe_dots: allocation failed");
    }
    std::vector<float> out(P / d.K * d.D);
    int ok = hipMemset(du, 0x80, 4 * nu) == hipSuccess && hipMemset(dd, 0x80, 4 * nd) == hipSuccess;
    if (ok) {
        g_dbg_up = du;
        g_dbg_dn = dd;
        ok = forward_host(L, in, out.data(), S, nullptr, nullptr);
        g_dbg_up = g_dbg_dn = nullptr;
    }
    ok = ok && hipMemcpy(up, du, 4 * nu, hipMemcpyDeviceToHost) == hipSuccess &&
         hipMemcpy(down, dd, 4 * nd, hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(du);
    (void)hipFree(dd);
    if (!ok) ZZ_FAIL("zz_moe_dots: forward failed");
    return 1;
}

extern "C" int zz_moe_forward_begin(int id, const float *in, int S) {
    Layer *L = get_layer(id);
    if (!L || !in || S <= 0) ZZ_FAIL("zz_moe_forward_begin: bad arguments");
    const zz_moe_desc &d = L->d;
    if (S > chunk_tokens(d)) ZZ_FAIL("zz_moe_forward_begin: S > %d", chunk_tokens(d));
    if (L->pending_S >= 0) ZZ_FAIL("zz_moe_forward_begin: a forward is already pending");
    if (L->n_present != d.E) ZZ_FAIL("forward: %d of %d experts uploaded", L->n_present, d.E);
    if (!ensure_ws(L, S)) return 0;
    ZZ_CHECK(hipMemcpyAsync(L->ws.in, in, sizeof(float) * S * d.D, hipMemcpyHostToDevice, g_stream));
    if (!run_chunk(L, L->ws, L->ws.in, L->ws.out, S, g_stream)) return 0;
    L->pending_S = S;
    return 1;
}

extern "C" int zz_moe_forward_end(int id, float *out, int *eidx, float *ewt) {
    Layer *L = get_layer(id);
    if (!L || L->pending_S < 0 || !out) ZZ_FAIL("zz_moe_forward_end: nothing pending");
    const zz_moe_desc &d = L->d;
    int S = L->pending_S;
    L->pending_S = -1;
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    ZZ_CHECK(hipMemcpy(out, L->ws.out, sizeof(float) * S * d.D, hipMemcpyDeviceToHost));
    if (eidx) ZZ_CHECK(hipMemcpy(eidx, L->ws.eidx, sizeof(int) * S * d.K, hipMemcpyDeviceToHost));
    if (ewt) ZZ_CHECK(hipMemcpy(ewt, L->ws.ewt, sizeof(float) * S * d.K, hipMemcpyDeviceToHost));
    return 1;
}

extern "C" int zz_moe_debug(int id, zz_moe_dump *dp) {
    Layer *L = get_layer(id);
    if (!L || !dp || L->last_S <= 0) ZZ_FAIL("zz_moe_debug: no forward to dump");
    const zz_moe_desc &d = L->d;
    Workspace &w = L->ws;
    const int S = L->last_S, P = S * d.K;
    const bool dec = L->last_dec;
    ZZ_CHECK(hipDeviceSynchronize());              // the forward may have run on any stream
    if (dec) {
        // the decode path routes inside its gate/up kernel and keeps the hidden by
        // flat pair: the dispatch lists are built here, from its routing outputs
        ZzDispatchArgs da;
        da.P = P; da.E = d.E; da.K = d.K; da.tch = ZZ_DEC_MAXS; da.eidx = w.eidx; da.ewt = w.ewt;
        da.xslots = zz_item_slots(d.E, P, S, ZZ_DEC_MAXS); da.wcost = zz_weight_cost(L->lay, d);
        da.ptok = w.ptok; da.pslot = w.pslot; da.pwt = w.pwt; da.ppos = w.ppos; da.uniq = w.uniq;
        da.uoff = w.uoff; da.ucnt = w.ucnt; da.items = w.items; da.meta = w.meta;
        if (!zz_launch_dispatch(da, g_stream)) ZZ_FAIL("zz_moe_debug: dispatch launch failed");
    }
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    if (dp->logits) {
        // the decode path keeps gemma's logits as centres with bounds only
        if ((dec && d.gating == ZZ_GATE_SOFTMAX_PES) || d.gating == ZZ_GATE_DENSE)
            ZZ_FAIL("zz_moe_debug: no router logits on this path");
        ZZ_CHECK(hipMemcpy(dp->logits, w.cen, sizeof(double) * S * d.E, hipMemcpyDeviceToHost));
    }
    if (dp->xq) ZZ_CHECK(hipMemcpy(dp->xq, w.xq, (size_t)S * d.D, hipMemcpyDeviceToHost));
    if (dp->xs) ZZ_CHECK(hipMemcpy(dp->xs, w.xs, sizeof(float) * S * (d.D / ZZ_BLK), hipMemcpyDeviceToHost));
    std::vector<int> ptok(P), pslot(P), ppos(P), meta(2), uniq(d.E), uoff(d.E), ucnt(d.E);
    ZZ_CHECK(hipMemcpy(ptok.data(), w.ptok, sizeof(int) * P, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(pslot.data(), w.pslot, sizeof(int) * P, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(ppos.data(), w.ppos, sizeof(int) * P, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(meta.data(), w.meta, sizeof(int) * 2, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(uniq.data(), w.uniq, sizeof(int) * d.E, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(uoff.data(), w.uoff, sizeof(int) * d.E, hipMemcpyDeviceToHost));
    ZZ_CHECK(hipMemcpy(ucnt.data(), w.ucnt, sizeof(int) * d.E, hipMemcpyDeviceToHost));
    const int nu = meta[0];
    dp->nu = nu;
    if (dp->uniq) memcpy(dp->uniq, uniq.data(), sizeof(int) * nu);
    dp->nitems = dec ? 0 : meta[1];
    if (dp->items && dp->items_cap > 0 && dp->nitems > 0) {
        const int ni = dp->nitems < dp->items_cap ? dp->nitems : dp->items_cap;
        static_assert(sizeof(ZzItem) == 4 * sizeof(int), "items are copied as 4 ints");
        ZZ_CHECK(hipMemcpy(dp->items, w.items, sizeof(ZzItem) * ni, hipMemcpyDeviceToHost));
    }
    // lists in union order, as moe_apply_chunk walks them (gemma4.c:776-790)
    int n = 0;
    for (int u = 0; u < nu; u++) {
        if (dp->offs) dp->offs[u] = n;
        for (int i = 0; i < ucnt[u]; i++, n++) {
            if (dp->rows) dp->rows[n] = ptok[uoff[u] + i];
            if (dp->slots) dp->slots[n] = pslot[uoff[u] + i];
        }
    }
    if (dp->offs) dp->offs[nu] = n;
    const int nbM = d.MI / ZZ_BLK;
    if (dp->hq || dp->hs) {
        std::vector<int8_t> hq((size_t)P * d.MI);
        std::vector<float> hs((size_t)P * nbM);
        ZZ_CHECK(hipMemcpy(hq.data(), w.hq, hq.size(), hipMemcpyDeviceToHost));
        ZZ_CHECK(hipMemcpy(hs.data(), w.hs, sizeof(float) * hs.size(), hipMemcpyDeviceToHost));
        for (int f = 0; f < P; f++) {              // (token, slot) order
            int p = dec ? f : ppos[f];
            if (p < 0 || p >= P) ZZ_FAIL("zz_moe_debug: pair %d of the last forward out of range", p);
            if (dp->hq) memcpy(dp->hq + (size_t)f * d.MI, hq.data() + (size_t)p * d.MI, d.MI);
            if (dp->hs) memcpy(dp->hs + (size_t)f * nbM, hs.data() + (size_t)p * nbM, sizeof(float) * nbM);
        }
    }
    return 1;
}

extern "C" int zz_moe_blockdots(int id, int eid, int tensor, int row0, int nrows, const int8_t *xq,
                                int32_t *out) {
    Layer *L = get_layer(id);
    if (!L || eid < 0 || eid >= L->d.E || tensor < 0 || tensor > 2 || !xq || !out) ZZ_FAIL("blockdots: bad arguments");
    ZzTensor t = tensor == 0 ? L->lay.gate : tensor == 1 ? L->lay.up : L->lay.down;
    if (row0 < 0 || nrows <= 0 || row0 + nrows > t.O) ZZ_FAIL("blockdots: rows out of range");
    int8_t *dx = nullptr;
    int32_t *dout = nullptr;
    size_t nout = (size_t)nrows * (t.I / ZZ_BLK);
    ZZ_CHECK(hipMalloc(&dx, t.I));
    if (hipMalloc(&dout, sizeof(int32_t) * nout) != hipSuccess) { (void)hipFree(dx); ZZ_FAIL("blockdots: alloc"); }
    int ok = hipMemcpy(dx, xq, t.I, hipMemcpyHostToDevice) == hipSuccess &&
             zz_launch_blockdots(L->slots + (size_t)eid * L->lay.bytes, t, row0, nrows, dx, dout, g_stream) &&
             hipStreamSynchronize(g_stream) == hipSuccess &&
             hipMemcpy(out, dout, sizeof(int32_t) * nout, hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dx);
    (void)hipFree(dout);
    if (!ok) ZZ_FAIL("blockdots: failed");
    return 1;
}

extern "C" int zz_quantize(int fmt, const float *d_w, uint8_t *d_out, int64_t n, void *stream) {
    if (!g_ready || !d_w || !d_out || n <= 0 || n % ZZ_BLK) ZZ_FAIL("zz_quantize: bad arguments");
    if (fmt != ZZ_FMT_Q40 && fmt != ZZ_FMT_Q80) ZZ_FAIL("zz_quantize: fmt %d declined", fmt);
    if (!zz_launch_quantize(fmt, d_w, d_out, n / ZZ_BLK, stream ? (hipStream_t)stream : g_stream))
        ZZ_FAIL("zz_quantize: launch failed");
    return 1;
}

extern "C" int zz_router_expf(const float *d_x, float *d_y, int64_t n, void *stream) {
    if (!g_ready || !d_x || !d_y || n <= 0) ZZ_FAIL("zz_router_expf: bad arguments");
    if (!zz_launch_expf(d_x, d_y, n, stream ? (hipStream_t)stream : g_stream)) ZZ_FAIL("zz_router_expf: launch failed");
    return 1;
}

extern "C" int zz_moe_stats(unsigned *c) {
    if (!g_ready || !c) ZZ_FAIL("zz_moe_stats: not ready");
    ZZ_CHECK(hipStreamSynchronize(g_stream));
    ZZ_CHECK(hipMemcpy(c, g_diag, 4 * sizeof(unsigned), hipMemcpyDeviceToHost));
    return 1;
}

extern "C" const char *zz_last_error(void) { return g_err; }

void zz_gemma_shutdown();   // zz_gemma.hip

extern "C" void gpu_shutdown(void) {
    if (!g_ready) return;
    (void)hipStreamSynchronize(g_stream);
    zz_gemma_shutdown();
    for (Layer *&L : g_layers) { free_layer(L); L = nullptr; }
    g_layers.clear();
    g_maps.clear([](const ZzRange &m) { (void)hipFree(m.dev); });
    if (g_mx) (void)hipFree(g_mx);
    if (g_my) (void)hipFree(g_my);
    g_mx = g_my = nullptr;
    g_mxn = g_myn = 0;
    (void)hipFree(g_diag);
    g_diag = nullptr;
    (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    g_ready = 0;
    snprintf(g_name, sizeof g_name, "none");
}
