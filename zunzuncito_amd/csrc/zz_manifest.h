// zz_manifest.h -- the container manifest and the host-range registry, host-only
// C++ (no HIP), so that tests/host_check.cpp builds them with g++ under ASAN/UBSAN.
//
// manifest.txt is the line grammar that tools/convert_*.py write and the engines
// read (gemma4.c:270-330, lfm25.c:290-350, maple.c:220-278, ling.c:270-336):
//   cfg <key> <value...>                  model configuration
//   esz <record> <gate bytes> <down bytes>  one record size for every layer (gemma, maple)
//   eszl <layer> <record> <gate> <down> <fmt>  per layer, with its expert format (lfm, ling)
//   dense <name> <offset> <length> <fmt> <O> <I>  a dense.bin tensor
//   expert <layer> <expert> <offset>      an experts.bin record
// Other lines (ndense, nexpert counts) are skipped, as the engines skip what they do
// not use. Unlike the engines, values that cannot be sizes or indices (negative, or
// past what the loader can address) fail the parse with a message.
#pragma once

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <string>
#include <utility>
#include <vector>

namespace zzm {

struct DenseEnt {
    int64_t off = 0, len = 0;
    int fmt = 0, O = 0, I = 0;        // fmt: 0 f32, 1 q4_0, 5 i32 (convert_gemma4.py:404)
};

struct RecSize {
    int64_t esz = 0, gate_b = 0, down_b = 0;
    int fmt = 0;                      // eszl: the layer's expert format; esz: 0 (not stated)
};

struct Manifest {
    std::map<std::string, std::string> cfg;
    RecSize all;                                   // `esz`
    std::map<int, RecSize> per_layer;              // `eszl`
    std::map<std::string, DenseEnt> dense;
    std::map<std::pair<int, int>, int64_t> eoff;   // (layer, expert) -> experts.bin offset

    int geti(const char *k, int dflt = -1) const {
        auto it = cfg.find(k);
        return it == cfg.end() ? dflt : atoi(it->second.c_str());
    }
    double getf(const char *k, double dflt = 0.0) const {
        auto it = cfg.find(k);
        return it == cfg.end() ? dflt : atof(it->second.c_str());
    }
    // the record size of layer li: its eszl line, else the esz line, else null
    const RecSize *rec(int li) const {
        auto it = per_layer.find(li);
        if (it != per_layer.end()) return &it->second;
        return all.esz > 0 ? &all : nullptr;
    }
};

// Parses the manifest text of one file. False with a message in err when the file
// cannot be read or a line holds a value that cannot be what it names.
inline bool parse_manifest(const std::string &path, Manifest &m, std::string &err) {
    FILE *f = fopen(path.c_str(), "r");
    if (!f) {
        err = "cannot open " + path;
        return false;
    }
    char line[4096];
    int ln = 0;
    bool ok = true;
    auto bad = [&](const char *what) {
        err = path + ":" + std::to_string(ln) + ": " + what;
        ok = false;
    };
    const int64_t lim = (int64_t)1 << 50;          // no offset or size reaches a petabyte
    while (ok && fgets(line, sizeof line, f)) {
        ln++;
        const size_t n = strlen(line);
        if (n == sizeof line - 1 && line[n - 1] != '\n') {   // longer than the buffer
            int c;
            while ((c = fgetc(f)) != EOF && c != '\n') {     // the rest is dropped
            }
            if (strncmp(line, "cfg ", 4) != 0) {   // only a cfg value (a list) may be that long;
                bad("line too long");              // it is kept cut at the buffer
                break;
            }
        }
        char k[128], nm[256];
        long long a, b, c, off, len;
        int li, e, fmt, O, I;
        if (sscanf(line, "cfg %127s", k) == 1) {
            const char *v = line + 4 + strlen(k);
            while (*v == ' ') v++;
            std::string val(v);
            while (!val.empty() && (val.back() == '\n' || val.back() == '\r')) val.pop_back();
            m.cfg[k] = val;
        } else if (sscanf(line, "eszl %d %lld %lld %lld %d", &li, &a, &b, &c, &fmt) == 5) {
            if (li < 0 || a <= 0 || b < 0 || c < 0 || a > lim || b > a || c > a) bad("bad eszl");
            else m.per_layer[li] = RecSize{a, b, c, fmt};
        } else if (sscanf(line, "esz %lld %lld %lld", &a, &b, &c) == 3) {
            if (a <= 0 || b < 0 || c < 0 || a > lim || b > a || c > a) bad("bad esz");
            else m.all = RecSize{a, b, c, 0};
        } else if (sscanf(line, "dense %255s %lld %lld %d %d %d", nm, &off, &len, &fmt, &O, &I) == 6) {
            if (off < 0 || len < 0 || off > lim || len > lim || O < 0 || I < 0) bad("bad dense entry");
            else {
                DenseEnt d;
                d.off = off;
                d.len = len;
                d.fmt = fmt;
                d.O = O;
                d.I = I;
                m.dense[nm] = d;
            }
        } else if (sscanf(line, "expert %d %d %lld", &li, &e, &off) == 3) {
            if (li < 0 || e < 0 || off < 0 || off > lim) bad("bad expert entry");
            else m.eoff[{li, e}] = off;
        }
    }
    fclose(f);
    return ok;
}

}  // namespace zzm

// -------------------------------------------------------------------------------
// The registry of host ranges that gpu_map has copied into device memory
// (gpu.h:66-69): a lookup finds the newest mapping that holds a range; mapping a range
// inside an existing mapping refreshes those bytes in place; a range that only
// overlaps older mappings replaces them (the host memory was released and reused).
// Arithmetic on addresses is done on uintptr_t with overflow checks: a range that
// would wrap the address space is inside no mapping, and overlaps those up to the top.
// Each mapping also keeps a sampled fingerprint of the host bytes it last uploaded:
// the 8 bytes at every multiple of ZZ_FP_STRIDE from its start. The engines map an
// expert slot once and later pread other experts into it (gemma4.c:2051-2058,
// 484-491); a matmul whose tensor's samples no longer match re-uploads that tensor
// first. An expert record read over another differs in essentially every sample; a
// rewrite that changes none of them (or a tensor shorter than the stride holding no
// sample) is not seen.
#define ZZ_FP_STRIDE 256
struct ZzRange {
    uintptr_t host;
    size_t n;
    uint8_t *dev;
    std::vector<uint64_t> fp;      // sample k: host bytes [k*STRIDE, k*STRIDE + 8)
};

// sample indices [*k0, *k1) that lie wholly inside [off, off + len) of a mapping
static inline void zz_fp_span(size_t off, size_t len, size_t *k0, size_t *k1) {
    *k0 = off / ZZ_FP_STRIDE + (off % ZZ_FP_STRIDE != 0);
    *k1 = len >= 8 ? (off + len - 8) / ZZ_FP_STRIDE + 1 : *k0;
    if (*k1 < *k0) *k1 = *k0;
}
// record the samples of [off, off + len) from the host bytes (after an upload of them)
static inline void zz_fp_take(ZzRange &m, size_t off, size_t len) {
    if (m.fp.empty() && m.n >= 8) m.fp.resize((m.n - 8) / ZZ_FP_STRIDE + 1);
    size_t k0, k1;
    zz_fp_span(off, len, &k0, &k1);
    for (size_t k = k0; k < k1 && k < m.fp.size(); k++)
        memcpy(&m.fp[k], (const void *)(m.host + k * ZZ_FP_STRIDE), 8);
}
// whether a sample of [off, off + len) differs from the host bytes now
static inline bool zz_fp_changed(const ZzRange &m, size_t off, size_t len) {
    size_t k0, k1;
    zz_fp_span(off, len, &k0, &k1);
    for (size_t k = k0; k < k1 && k < m.fp.size(); k++) {
        uint64_t w;
        memcpy(&w, (const void *)(m.host + k * ZZ_FP_STRIDE), 8);
        if (w != m.fp[k]) return true;
    }
    return false;
}

class ZzRanges {
    std::vector<ZzRange> v_;

    static bool inside(const ZzRange &m, uintptr_t q, size_t n) {
        return n <= m.n && q >= m.host && q - m.host <= m.n - n;
    }
    static bool overlaps(const ZzRange &m, uintptr_t q, size_t n) {
        if (n == 0 || m.n == 0) return false;
        // ends saturate at the top of the address space instead of wrapping
        const uintptr_t qe = n > UINTPTR_MAX - q ? UINTPTR_MAX : q + n;
        const uintptr_t me = m.n > UINTPTR_MAX - m.host ? UINTPTR_MAX : m.host + m.n;
        return q < me && m.host < qe;
    }

public:
    // the newest mapping that holds [p, p + n), or null
    const ZzRange *find(const void *p, size_t n) const {
        const uintptr_t q = (uintptr_t)p;
        for (size_t i = v_.size(); i-- > 0;)
            if (inside(v_[i], q, n)) return &v_[i];
        return nullptr;
    }
    ZzRange *find(const void *p, size_t n) { return const_cast<ZzRange *>(((const ZzRanges *)this)->find(p, n)); }
    // removes every mapping that overlaps [p, p + n), handing each to drop(ZzRange)
    template <class F>
    void drop_overlaps(const void *p, size_t n, F drop) {
        const uintptr_t q = (uintptr_t)p;
        for (size_t i = v_.size(); i-- > 0;)
            if (overlaps(v_[i], q, n)) {
                drop(v_[i]);
                v_.erase(v_.begin() + (long)i);
            }
    }
    ZzRange &add(const void *p, size_t n, uint8_t *dev) {
        v_.push_back(ZzRange{(uintptr_t)p, n, dev, {}});
        return v_.back();
    }
    template <class F>
    void clear(F drop) {
        for (ZzRange &m : v_) drop(m);
        v_.clear();
    }
    size_t size() const { return v_.size(); }
};
