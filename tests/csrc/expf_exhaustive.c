/* Exhaustive comparison of the device expf restatement (compiled here for the
 * host; the branching, the branch-free and, on its domain, the non-positive
 * form) with the host libm expf over every float bit pattern in [lo, hi).
 * Usage: expf_exhaustive FORM_UNUSED lo hi   (the form is fixed at compile time)
 * Prints: "<mismatches> <first mismatching bits or -1>". */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <xmmintrin.h>

#include "kvexp_expf.h"

int main(int argc, char **argv) {
    unsigned long long lo = argc > 1 ? strtoull(argv[1], 0, 0) : 0;
    unsigned long long hi = argc > 2 ? strtoull(argv[2], 0, 0) : (1ull << 32);
    _mm_setcsr(_mm_getcsr() & ~((1u << 15) | (1u << 6)));
    unsigned long long bad = 0;
    long long first = -1;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 20)
    for (long long u = (long long)lo; u < (long long)hi; ++u) {
        _mm_setcsr(_mm_getcsr() & ~((1u << 15) | (1u << 6)));
        uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        float a = expf(x), d = kvexp_expf(x), e = kvexp_expf_tab_nb(x, kvexp_exp2_32_table);
        /* the non-positive form: x <= 0 (sign bit set), +0 and NaN only */
        const int np = (b >> 31) || b == 0u || isnan(x);
        float f = np ? kvexp_expf_nonpos_nb(x, kvexp_exp2_32_table) : a;
        uint32_t ua, ud, ue, uf;
        memcpy(&ua, &a, 4);
        memcpy(&ud, &d, 4);
        memcpy(&ue, &e, 4);
        memcpy(&uf, &f, 4);
        if ((ua != ud && !(isnan(a) && isnan(d))) || (ua != ue && !(isnan(a) && isnan(e))) ||
            (ua != uf && !(isnan(a) && isnan(f)))) {
            ++bad;
#pragma omp critical
            if (first < 0 || u < first) first = u;
        }
    }
    printf("%llu %lld\n", bad, first);
    return 0;
}
