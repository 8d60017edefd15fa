// zz_container.hip -- zunzuncito container directories into HBM (host code):
//   zz_moe_load_experts: one layer's expert records from experts.bin into the layer's
//     slot table (every expert resident: no slot/LRU tier, no I/O threads);
//   zz_gemma_stack_load: a whole gemma4 container as a resident stack.
// The container is what tools/convert_*.py write and gemma4.c:260-403 /
// lfm25.c:280-420 read: manifest.txt (cfg lines, the record size, the dense tensor
// index, one offset per expert), dense.bin (tensors back to back, q4_0 matrices and
// f32 vectors) and experts.bin (4096-aligned [gate | up | down] records).
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_manifest.h"
#include "../../include/zz_gemma.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <map>
#include <string>
#include <utility>
#include <vector>

#define ZZ_FAIL(...)               \
    do {                           \
        zz_set_error(__VA_ARGS__); \
        return 0;                  \
    } while (0)

int zz_stack_adopt(int id, const std::vector<int> &layers, const std::vector<int> &blocks, int head);

namespace {

using zzm::DenseEnt;
using zzm::Manifest;
using zzm::RecSize;

int parse_manifest(const std::string &dir, Manifest &m) {
    std::string err;
    if (!zzm::parse_manifest(dir + "/manifest.txt", m, err)) ZZ_FAIL("container: %s", err.c_str());
    return 1;
}

int read_at(int fd, int64_t off, int64_t len, void *dst) {
    uint8_t *p = (uint8_t *)dst;
    for (int64_t done = 0; done < len;) {
        const ssize_t r = pread(fd, p + done, (size_t)(len - done), (off_t)(off + done));
        if (r <= 0) return 0;
        done += r;
    }
    return 1;
}

struct Fd {
    int fd = -1;
    explicit Fd(const std::string &p) : fd(open(p.c_str(), O_RDONLY)) {}
    ~Fd() {
        if (fd >= 0) close(fd);
    }
};

int load_experts(int layer, const std::string &dir, const Manifest &m, int li) {
    const zz_moe_desc *d = zz_layer_desc(layer);
    if (!d) ZZ_FAIL("zz_moe_load_experts: no such layer");
    const RecSize *rs = m.rec(li);
    if (!rs) ZZ_FAIL("zz_moe_load_experts: manifest has no record size for layer %d", li);
    const int64_t want = zz_moe_record_bytes(d);
    if (rs->esz != want)
        ZZ_FAIL("zz_moe_load_experts: container records are %lld bytes, the layer's %lld", (long long)rs->esz,
                (long long)want);
    // an eszl layer states its expert format, one for all three tensors (lfm25.c:328-331,
    // convert_lfm25.py's expert_fmt): the layer must read its records that way
    if (rs->fmt && (d->fmt_gate != rs->fmt || d->fmt_up != rs->fmt || d->fmt_down != rs->fmt))
        ZZ_FAIL("zz_moe_load_experts: layer %d's records are format %d, the layer's (%d, %d, %d)", li, rs->fmt,
                d->fmt_gate, d->fmt_up, d->fmt_down);
    Fd f(dir + "/experts.bin");
    if (f.fd < 0) ZZ_FAIL("zz_moe_load_experts: cannot open %s/experts.bin", dir.c_str());
    std::vector<uint8_t> rec((size_t)rs->esz);
    for (int e = 0; e < d->E; e++) {
        auto it = m.eoff.find({li, e});
        if (it == m.eoff.end()) ZZ_FAIL("zz_moe_load_experts: no expert %d of layer %d", e, li);
        if (!read_at(f.fd, it->second, rs->esz, rec.data()))
            ZZ_FAIL("zz_moe_load_experts: short read of expert %d of layer %d", e, li);
        if (!zz_moe_expert_upload(layer, e, rec.data(), rec.size())) return 0;
    }
    return 1;
}

// one dense tensor of the expected format and element count, read from dense.bin
int dense_read(int fd, const Manifest &m, const std::string &name, int fmt, int64_t len, std::vector<uint8_t> &out) {
    auto it = m.dense.find(name);
    if (it == m.dense.end()) ZZ_FAIL("container: missing dense tensor %s", name.c_str());
    if (it->second.fmt != fmt || it->second.len != len)
        ZZ_FAIL("container: dense tensor %s is fmt %d, %lld bytes (want fmt %d, %lld)", name.c_str(),
                it->second.fmt, (long long)it->second.len, fmt, (long long)len);
    out.resize((size_t)len);
    if (!read_at(fd, it->second.off, len, out.data())) ZZ_FAIL("container: short read of %s", name.c_str());
    return 1;
}

}  // namespace

extern "C" int zz_moe_load_experts(int layer, const char *dir, int li) {
    if (!zz_lib_ready() || !dir) ZZ_FAIL("zz_moe_load_experts: not ready or no directory");
    Manifest m;
    if (!parse_manifest(dir, m)) return 0;
    return load_experts(layer, dir, m, li);
}

extern "C" int zz_gemma_stack_load(const char *dir_c, int *n_layers_out, int *D_out, int *V_out) {
    if (!zz_lib_ready() || !dir_c) {
        zz_set_error("zz_gemma_stack_load: not ready or no directory");
        return -1;
    }
    const std::string dir(dir_c);
    Manifest m;
    if (!parse_manifest(dir, m)) return -1;
    const int D = m.geti("hidden"), NL = m.geti("n_layers"), E = m.geti("n_experts"), K = m.geti("topk");
    const int MI = m.geti("moe_inter"), DI = m.geti("dense_inter"), V = m.geti("vocab");
    const float eps = (float)m.getf("eps", 1e-6), escale = (float)m.getf("embed_scale", 1.0);
    const float cap = (float)m.getf("final_logit_softcap", 0.0);
    if (D <= 0 || NL <= 0 || E <= 0 || K <= 0 || MI <= 0 || DI <= 0 || V <= 0) {
        zz_set_error("zz_gemma_stack_load: manifest lacks hidden / n_layers / n_experts / topk / moe_inter / "
                     "dense_inter / vocab");
        return -1;
    }
    Fd f(dir + "/dense.bin");
    if (f.fd < 0) {
        zz_set_error("zz_gemma_stack_load: cannot open %s/dense.bin", dir.c_str());
        return -1;
    }
    const int64_t q40 = 18;
    auto qbytes = [&](int O, int I) { return (int64_t)O * (I / ZZ_BLK) * q40; };
    std::vector<int> layers, blocks;
    int head = -1;
    auto fail = [&]() {
        for (int b : blocks) zz_ffn_block_destroy(b);
        for (int l : layers) zz_moe_layer_destroy(l);
        if (head >= 0) zz_head_destroy(head);
        return -1;
    };
    std::vector<uint8_t> router, rscale, pes, pre2, post2, pre, post1, post, ls, g, u, dn;
    for (int l = 0; l < NL; l++) {
        const std::string o = "layers." + std::to_string(l) + ".";
        if (!dense_read(f.fd, m, o + "router_proj", 0, (int64_t)E * D * 4, router) ||
            !dense_read(f.fd, m, o + "router_scale", 0, (int64_t)D * 4, rscale) ||
            !dense_read(f.fd, m, o + "router_pes", 0, (int64_t)E * 4, pes) ||
            !dense_read(f.fd, m, o + "pre_feedforward_layernorm_2", 0, (int64_t)D * 4, pre2) ||
            !dense_read(f.fd, m, o + "post_feedforward_layernorm_2", 0, (int64_t)D * 4, post2) ||
            !dense_read(f.fd, m, o + "pre_feedforward_layernorm", 0, (int64_t)D * 4, pre) ||
            !dense_read(f.fd, m, o + "post_feedforward_layernorm_1", 0, (int64_t)D * 4, post1) ||
            !dense_read(f.fd, m, o + "post_feedforward_layernorm", 0, (int64_t)D * 4, post) ||
            !dense_read(f.fd, m, o + "layer_scalar", 0, 4, ls) ||
            !dense_read(f.fd, m, o + "mlp_gate", 1, qbytes(DI, D), g) ||
            !dense_read(f.fd, m, o + "mlp_up", 1, qbytes(DI, D), u) ||
            !dense_read(f.fd, m, o + "mlp_down", 1, qbytes(D, DI), dn))
            return fail();
        zz_moe_desc md;
        memset(&md, 0, sizeof md);
        md.D = D; md.MI = MI; md.E = E; md.K = K;
        md.gating = ZZ_GATE_SOFTMAX_PES; md.act = ZZ_ACT_GEGLU_TANH;
        md.fmt_gate = md.fmt_up = md.fmt_down = ZZ_FMT_Q40;
        md.norm_topk = 1; md.eps = eps; md.routed_scaling = 1.0f; md.clamp = 0.0f;
        zz_moe_weights mw;
        memset(&mw, 0, sizeof mw);
        mw.router = (const float *)router.data();
        mw.router_scale = (const float *)rscale.data();
        mw.pes = (const float *)pes.data();
        mw.pre_ln = (const float *)pre2.data();
        mw.post_ln = (const float *)post2.data();
        const int moe = zz_moe_layer_create(&md, &mw);
        if (moe < 0) return fail();
        layers.push_back(moe);
        if (!load_experts(moe, dir, m, l)) return fail();
        // the dense MLP as a one-expert record mlp_gate | mlp_up | mlp_down
        zz_moe_desc dd = md;
        dd.MI = DI; dd.E = 1; dd.K = 1; dd.gating = ZZ_GATE_DENSE;
        zz_moe_weights dw;
        memset(&dw, 0, sizeof dw);
        dw.pre_ln = (const float *)pre.data();
        dw.post_ln = (const float *)post1.data();
        const int den = zz_moe_layer_create(&dd, &dw);
        if (den < 0) return fail();
        layers.push_back(den);
        std::vector<uint8_t> rec;
        rec.reserve(g.size() + u.size() + dn.size());
        rec.insert(rec.end(), g.begin(), g.end());
        rec.insert(rec.end(), u.begin(), u.end());
        rec.insert(rec.end(), dn.begin(), dn.end());
        if (!zz_moe_expert_upload(den, 0, rec.data(), rec.size())) return fail();
        float scalar;
        memcpy(&scalar, ls.data(), 4);
        const int b = zz_ffn_block_create(moe, den, (const float *)post.data(), scalar);
        if (b < 0) return fail();
        blocks.push_back(b);
    }
    std::vector<uint8_t> table, fnorm;
    if (!dense_read(f.fd, m, "embed_tokens", 1, qbytes(V, D), table) ||
        !dense_read(f.fd, m, "norm", 0, (int64_t)D * 4, fnorm))
        return fail();
    head = zz_head_create(table.data(), V, D, (const float *)fnorm.data(), eps, escale, cap);
    if (head < 0) return fail();
    const int NC = m.geti("flash_n_clusters", 0);
    if (NC > 0) {                                // a FlashHead: gemma4.c:302-306, 357-362
        const int CS = m.geti("flash_cluster_size"), NP = m.geti("flash_n_probes");
        const int nf = m.geti("flash_n_force", 0), scaled = m.geti("flash_scaled_centroids", 0);
        std::vector<uint8_t> cent, tmap, cs, fo;
        if (CS <= 0 || NP <= 0 || nf < 0 || !dense_read(f.fd, m, "flash_centroids", 1, qbytes(NC, D), cent) ||
            !dense_read(f.fd, m, "flash_token_map", 5, (int64_t)NC * CS * 4, tmap) ||
            !dense_read(f.fd, m, "flash_cluster_scale", 0, (int64_t)NC * 4, cs) ||
            !dense_read(f.fd, m, "flash_force", 5, (int64_t)(nf > 0 ? nf : 1) * 4, fo) ||
            !zz_head_flash(head, cent.data(), NC, (const int32_t *)tmap.data(), CS, NP, (const float *)cs.data(),
                           scaled, (const int32_t *)fo.data(), nf))
            return fail();
    }
    const int stack = zz_stack_create(blocks.data(), (int)blocks.size(), head);
    if (stack < 0 || !zz_stack_adopt(stack, layers, blocks, head)) return fail();
    if (n_layers_out) *n_layers_out = NL;
    if (D_out) *D_out = D;
    if (V_out) *V_out = V;
    return stack;
}
