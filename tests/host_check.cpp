// host_check.cpp -- host-only checks of the container manifest parser and of the
// gpu_map range registry (zunzuncito_amd/csrc/zz_manifest.h, both compiled into
// libzzmoe.so). tests/Makefile builds this with g++ twice: plain, and under
// AddressSanitizer + UndefinedBehaviorSanitizer with recovery off, so that any
// out-of-bounds access, leak or undefined operation in that code ends the run.
//
//   host_check <scratch directory>
#include "../zunzuncito_amd/csrc/zz_manifest.h"

#include <stdio.h>
#include <string>

static int fails = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);      \
            fails++;                                                          \
        }                                                                     \
    } while (0)

static std::string g_dir;

static std::string put(const std::string &name, const std::string &text) {
    const std::string p = g_dir + "/" + name;
    FILE *f = fopen(p.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "cannot write %s\n", p.c_str());
        exit(2);
    }
    fwrite(text.data(), 1, text.size(), f);
    fclose(f);
    return p;
}

static bool parse(const std::string &text, zzm::Manifest &m, std::string &err) {
    return zzm::parse_manifest(put("manifest.txt", text), m, err);
}

static void manifests() {
    std::string err;
    {   // gemma / maple form: one record size, dense index, expert offsets (convert_gemma4.py)
        zzm::Manifest m;
        CHECK(parse("cfg hidden 2816\ncfg eps 1e-06\ncfg layer_types 0 1 0 0\n"
                    "esz 3340800 1115136 1110528\nndense 2\n"
                    "dense embed_tokens 0 831520 1 2816 262144\ndense norm 831520 11264 0 2816 1\n"
                    "nexpert 2\nexpert 0 0 0\nexpert 0 1 3342336\n", m, err));
        CHECK(m.geti("hidden") == 2816 && m.getf("eps") == 1e-6 && m.cfg["layer_types"] == "0 1 0 0");
        CHECK(m.all.esz == 3340800 && m.all.gate_b == 1115136 && m.all.down_b == 1110528 && m.all.fmt == 0);
        CHECK(m.dense.size() == 2 && m.dense["norm"].off == 831520 && m.dense["embed_tokens"].I == 262144);
        CHECK(m.eoff.size() == 2 && m.eoff[std::make_pair(0, 1)] == 3342336);
        CHECK(m.rec(7) == &m.all && m.geti("missing", 5) == 5);
    }
    {   // lfm / ling form: a record size and expert format per layer (convert_lfm25.py:490)
        zzm::Manifest m;
        CHECK(parse("cfg n_layers 3\neszl 0 100 30 40 1\neszl 2 200 60 80 2\r\nexpert 2 5 8192\n", m, err));
        CHECK(m.rec(0) && m.rec(0)->esz == 100 && m.rec(0)->fmt == 1);
        CHECK(m.rec(2) && m.rec(2)->gate_b == 60 && m.rec(2)->fmt == 2);
        CHECK(m.rec(1) == nullptr);                       // no eszl and no esz line
    }
    // values that cannot be sizes or indices fail with the line number
    const char *bad[] = {"esz 0 1 1\n", "esz 10 20 1\n", "eszl -1 100 30 40 1\n", "eszl 0 100 30 400 1\n",
                         "expert 0 -3 0\n", "expert 0 1 -4096\n", "dense w -1 10 1 2 3\n",
                         "dense w 0 10 1 -2 3\n", "esz 2000000000000000000 1 1\n"};
    for (const char *b : bad) {
        zzm::Manifest m;
        err.clear();
        CHECK(!parse(std::string("cfg hidden 8\n") + b, m, err));
        CHECK(err.find(":2:") != std::string::npos);
    }
    {   // a long cfg value (a list) is kept cut at the buffer; any other long line fails
        zzm::Manifest m;
        CHECK(parse("cfg layer_types " + std::string(9000, '1') + "\nesz 10 2 2\n", m, err));
        CHECK(m.all.esz == 10 && m.cfg["layer_types"].size() > 4000);
        zzm::Manifest m2;
        CHECK(!parse("expert 0 0 " + std::string(9000, '7') + "\n", m2, err));
    }
    {   // no file
        zzm::Manifest m;
        CHECK(!zzm::parse_manifest(g_dir + "/nonexistent/manifest.txt", m, err));
        CHECK(err.find("cannot open") != std::string::npos);
    }
    // random text built from the grammar's words and numbers, and raw bytes: any result,
    // but no crash and nothing out of bounds
    static const char *words[] = {"cfg", "esz", "eszl", "dense", "expert", "ndense", "nexpert", "-",
                                  "0", "-1", "4096", "99999999999999999999", "1e308", "x", "\t", " "};
    unsigned long long r = 12345;
    auto next = [&]() { return (unsigned)((r = r * 6364136223846793005ULL + 1442695040888963407ULL) >> 33); };
    for (int it = 0; it < 3000; it++) {
        std::string t;
        const int nl = (int)(next() % 12);
        for (int l = 0; l < nl; l++) {
            const int nw = (int)(next() % 9);
            for (int w = 0; w < nw; w++) {
                t += words[next() % 16];
                t += ' ';
            }
            if (next() % 7 == 0)
                for (int b = 0; b < (int)(next() % 64); b++) t += (char)(next() & 255);
            t += '\n';
        }
        zzm::Manifest m;
        (void)parse(t, m, err);
        for (auto &kv : m.per_layer) CHECK(kv.first >= 0 && kv.second.esz > 0);
        for (auto &kv : m.eoff) CHECK(kv.first.first >= 0 && kv.first.second >= 0 && kv.second >= 0);
    }
}

static void ranges() {
    static uint8_t buf[4096];
    uint8_t *A = (uint8_t *)0x1000, *B = (uint8_t *)0x2000, *C = (uint8_t *)0x3000;   // device stand-ins
    ZzRanges g;
    g.add(buf, 1000, A);
    CHECK(g.find(buf, 1000) && g.find(buf, 1000)->dev == A);
    CHECK(g.find(buf + 10, 50) && !g.find(buf + 990, 20) && !g.find(buf + 1000, 1));
    CHECK(g.find(buf + 1000, 0) != nullptr);          // an empty range at the end is inside
    g.add(buf + 100, 100, B);                         // a newer mapping nested in the first
    CHECK(g.find(buf + 150, 10)->dev == B && g.find(buf + 50, 10)->dev == A && g.find(buf + 150, 100)->dev == A);
    int dropped = 0;
    g.drop_overlaps(buf + 190, 20, [&](const ZzRange &m) { dropped += m.dev == A || m.dev == B; });
    CHECK(dropped == 2 && g.size() == 0);
    g.add(buf + 2000, 100, C);
    g.drop_overlaps(buf + 2100, 50, [&](const ZzRange &) { dropped++; });       // touching, not overlapping
    CHECK(dropped == 2 && g.size() == 1);
    // ranges at the top of the address space: no wrap, no undefined arithmetic
    const void *top = (const void *)(UINTPTR_MAX - 15);
    CHECK(g.find(top, 64) == nullptr && g.find((const void *)UINTPTR_MAX, 1) == nullptr);
    g.add(top, 8, A);
    CHECK(g.find(top, 8) != nullptr && g.find(top, 16) == nullptr);
    int n = 0;
    g.drop_overlaps(top, 64, [&](const ZzRange &) { n++; });
    CHECK(n == 1);
    g.clear([&](const ZzRange &) { n++; });
    CHECK(n == 2 && g.size() == 0);
}

// the sampled fingerprint of a mapping: taken after an upload, compared before use
static void fingerprints() {
    static uint8_t buf[10000];
    for (size_t i = 0; i < sizeof buf; i++) buf[i] = (uint8_t)(i * 131 + 7);
    uint8_t *A = (uint8_t *)0x1000;
    ZzRanges g;
    ZzRange &m = g.add(buf, sizeof buf, A);
    zz_fp_take(m, 0, sizeof buf);
    CHECK(m.fp.size() == (sizeof buf - 8) / ZZ_FP_STRIDE + 1);
    CHECK(!zz_fp_changed(m, 0, sizeof buf) && !zz_fp_changed(m, 300, 4000));
    buf[5 * ZZ_FP_STRIDE + 3] ^= 1;                 // inside sample 5
    CHECK(zz_fp_changed(m, 0, sizeof buf) && zz_fp_changed(m, 5 * ZZ_FP_STRIDE, 8));
    CHECK(!zz_fp_changed(m, 6 * ZZ_FP_STRIDE, 3000));           // a tensor after it: untouched
    CHECK(!zz_fp_changed(m, 5 * ZZ_FP_STRIDE + 1, 500));        // sample 5 not wholly inside
    zz_fp_take(m, 4 * ZZ_FP_STRIDE, 2 * ZZ_FP_STRIDE);          // that sub-range re-uploaded
    CHECK(!zz_fp_changed(m, 0, sizeof buf));
    buf[sizeof buf - 1] ^= 1;                       // past the last sample: not seen
    CHECK(!zz_fp_changed(m, 0, sizeof buf));
    buf[(m.fp.size() - 1) * ZZ_FP_STRIDE] ^= 1;     // the last sample
    CHECK(zz_fp_changed(m, 0, sizeof buf));
    // empty and short ranges: no sample, nothing read out of bounds
    CHECK(!zz_fp_changed(m, sizeof buf, 0) && !zz_fp_changed(m, sizeof buf - 7, 7));
    zz_fp_take(m, sizeof buf - 4, 4);
    static uint8_t tiny[5];
    ZzRange &t = g.add(tiny, sizeof tiny, A);
    zz_fp_take(t, 0, sizeof tiny);
    CHECK(t.fp.empty() && !zz_fp_changed(t, 0, sizeof tiny));
    g.clear([](const ZzRange &) {});
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s <scratch directory>\n", argv[0]);
        return 2;
    }
    g_dir = argv[1];
    manifests();
    ranges();
    fingerprints();
    printf("host_check %s (%d failures)\n", fails ? "FAILED" : "ok", fails);
    return fails ? 1 : 0;
}
