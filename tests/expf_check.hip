// expf_check.hip -- host-side check of zz_expf (zunzuncito_amd/csrc/zz_expf.h)
// against the host libm's expf (glibc) on inputs [lo, hi) of the 32-bit patterns
// (all 2^32 by default). Prints the number of mismatches; NaN matches NaN.
// Built and run by tests/test_expf.py; it makes no GPU call.
#include "../zunzuncito_amd/csrc/zz_expf.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int main(int argc, char **argv) {
    const long long lo = argc > 1 ? atoll(argv[1]) : 0, hi = argc > 2 ? atoll(argv[2]) : (1LL << 32);
    long long bad = 0;
    unsigned first = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (long long i = lo; i < hi; i++) {
        const unsigned u = (unsigned)i;
        float x;
        memcpy(&x, &u, 4);
        const float w = expf(x), g = zz_expf(x);
        unsigned uw, ug;
        memcpy(&uw, &w, 4);
        memcpy(&ug, &g, 4);
        if (uw != ug && !(w != w && g != g)) {
            bad++;
#pragma omp critical
            if (!first) first = u;
        }
    }
    printf("inputs %lld mismatches %lld first 0x%08x\n", hi - lo, bad, first);
    return bad != 0;
}
