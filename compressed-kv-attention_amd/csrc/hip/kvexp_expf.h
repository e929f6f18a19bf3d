/* Single-precision exp that returns glibc 2.35's expf bits.
 *
 * The reference computes every softmax coefficient with std::exp(float)
 * (src/softmax.hpp:10-11,20-21), i.e. glibc's expf. Matching the reference
 * output bit for bit on the GPU therefore needs the same function, so this
 * is a restatement of glibc 2.35's expf (sysdeps/ieee754/flt-32/e_expf.c,
 * the published ARM optimized-routines algorithm):
 *
 *   x * 32/ln2 = k + r, |r| <= 1/2, k integer (round to nearest even via the
 *   1.5*2^52 shift);
 *   exp(x) = 2^(k/32) * 2^(r/32) ~= s * (1 + C2 r + C1 r^2 + C0 r^3),
 *   s = 2^(k/32) read from a 32-entry table of 2^(i/32) rounded to double,
 *   stored minus (i << 47) so that adding k << 47 forms s directly.
 *
 * Evaluated in double precision, then rounded to float once. The table below
 * is 2^(i/32) correctly rounded, computed from first principles; C0..C2 are
 * the published minimax coefficients (scaled by 32^-3, 32^-2, 32^-1).
 *
 * glibc on x86-64 runs an FMA-compiled copy of this code on FMA-capable CPUs
 * (the __expf_fma ifunc variant); KVEXP_EXPF_FORM selects which operations are
 * fused so the result equals that build. An exhaustive comparison over all
 * 2^32 inputs against the host libm pins the choice (tests/test_expf.py).
 *
 *   form 0: no fused operation
 *   form 1: the three polynomial steps fused
 *   form 2: form 1, plus x*32/ln2 fused into both uses (shift add, remainder)
 *
 * The header compiles as C or C++ on the host (gcc) and as HIP device code.
 */
#ifndef KVEXP_EXPF_H
#define KVEXP_EXPF_H

#include <stdint.h>
#include <string.h>

#ifndef KVEXP_EXPF_FORM
#define KVEXP_EXPF_FORM 2
#endif

#if defined(__HIPCC__)
#define KVEXP_HD __host__ __device__ static inline __attribute__((always_inline))
#define KVEXP_EXP_TABLE_QUAL static __constant__ __device__
#else
#define KVEXP_HD static inline
#define KVEXP_EXP_TABLE_QUAL static const
#endif

#define KVEXP_EXP2_32_VALUES \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

KVEXP_EXP_TABLE_QUAL uint64_t kvexp_exp2_32_table[32] = {KVEXP_EXP2_32_VALUES};

#if defined(__HIPCC__)
/* Lane i < 32 of a wave stores table entry i at dst[i] (a copy in LDS). The
 * entries come from scalar immediates written into the lanes
 * (v_writelane_b32), not from a load of the table in global memory, so a
 * kernel that starts with this copy does not wait one or two memory round
 * trips (the table's address, then its bytes) before its first own loads.
 * Call with the whole wave active. */
template <int K>
__device__ static inline void kvexp_exp_table_lanes(uint32_t &lo, uint32_t &hi) {
    constexpr uint64_t t[32] = {KVEXP_EXP2_32_VALUES};
    asm("v_writelane_b32 %0, %1, %2" : "+v"(lo) : "s"(uint32_t(t[K])), "n"(K));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(hi) : "s"(uint32_t(t[K] >> 32)), "n"(K));
    if constexpr (K + 1 < 32) kvexp_exp_table_lanes<K + 1>(lo, hi);
}
__device__ static inline void kvexp_exp_table_to_lds(uint64_t *dst) {
    uint32_t lo = 0, hi = 0;
    kvexp_exp_table_lanes<0>(lo, hi);
    const int lane = int(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
    if (lane < 32) dst[lane] = (uint64_t(hi) << 32) | lo;
}
#endif


#define KVEXP_EXP_INVLN2N (0x1.71547652b82fep+0 * 32.0)
#define KVEXP_EXP_SHIFT 0x1.8p+52
#define KVEXP_EXP_C0 (0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0)
#define KVEXP_EXP_C1 (0x1.ebfce50fac4f3p-3 / 32.0 / 32.0)
#define KVEXP_EXP_C2 (0x1.62e42ff0c52d6p-1 / 32.0)

KVEXP_HD uint32_t kvexp_f32_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
KVEXP_HD uint64_t kvexp_f64_bits(double x) {
    uint64_t u;
    memcpy(&u, &x, 8);
    return u;
}
KVEXP_HD double kvexp_f64_from(uint64_t u) {
    double x;
    memcpy(&x, &u, 8);
    return x;
}

#define KVEXP_FMA64(a, b, c) __builtin_fma((a), (b), (c))

/* The reduction and polynomial, for |x| < 88 (no special case), reading
 * 2^(i/32) from `tab` (a copy of kvexp_exp2_32_table, e.g. in LDS). */
KVEXP_HD float kvexp_expf_core_tab(float x, const uint64_t *tab) {
    const double xd = (double)x;
#if KVEXP_EXPF_FORM >= 2
    double kd = KVEXP_FMA64(KVEXP_EXP_INVLN2N, xd, KVEXP_EXP_SHIFT);
    const uint64_t ki = kvexp_f64_bits(kd);
    kd -= KVEXP_EXP_SHIFT;
    const double r = KVEXP_FMA64(KVEXP_EXP_INVLN2N, xd, -kd);
#else
    const double z = KVEXP_EXP_INVLN2N * xd;
    double kd = z + KVEXP_EXP_SHIFT;
    const uint64_t ki = kvexp_f64_bits(kd);
    kd -= KVEXP_EXP_SHIFT;
    const double r = z - kd;
#endif
    /* s = tab[ki % 32] + (ki << 47): the shifted index has no bits in the
     * low word, so only the high word is added to (one 32-bit add). */
    const uint64_t tb = tab[ki & 31u];
    const uint32_t s_hi = (uint32_t)(tb >> 32) + ((uint32_t)ki << 15);
    const double s = kvexp_f64_from(((uint64_t)s_hi << 32) | (uint32_t)tb);
    const double r2 = r * r;
#if KVEXP_EXPF_FORM >= 1
    const double p = KVEXP_FMA64(KVEXP_EXP_C0, r, KVEXP_EXP_C1);
    double y = KVEXP_FMA64(KVEXP_EXP_C2, r, 1.0);
    y = KVEXP_FMA64(p, r2, y);
#else
    const double p = KVEXP_EXP_C0 * r + KVEXP_EXP_C1;
    double y = KVEXP_EXP_C2 * r + 1.0;
    y = p * r2 + y;
#endif
    return (float)(y * s);
}

/* expf with glibc's special cases: -inf -> +0, NaN/+inf -> x + x,
 * x > 0x1.62e42ep6 -> +inf, x < -0x1.9fe368p6 -> +0. */
KVEXP_HD float kvexp_expf_tab(float x, const uint64_t *tab) {
    const uint32_t ux = kvexp_f32_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    return kvexp_expf_core_tab(x, tab);
}

/* kvexp_expf_tab without branches: the reduction and polynomial run for every
 * input (the table index is always in range) and the special cases are
 * selected afterwards, so the result is the same for every x. */
KVEXP_HD float kvexp_expf_tab_nb(float x, const uint64_t *tab) {
    const float core = kvexp_expf_core_tab(x, tab);
    const uint32_t ux = kvexp_f32_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    float special = core;
    special = x < -0x1.9fe368p6f ? 0.0f : special;
    special = x > 0x1.62e42ep6f ? __builtin_inff() : special;
    special = abstop >= 0x7f8u ? x + x : special;
    special = ux == 0xff800000u ? 0.0f : special;
    return abstop >= 0x42bu ? special : core;
}

#if defined(__HIP_DEVICE_COMPILE__) && KVEXP_EXPF_FORM == 2
/* Device form of kvexp_expf_core_tab (form 2): the same operations in a fixed
 * instruction sequence. Left to itself the compiler rebuilds the table add
 * through 32-bit halves and copies constants for two-address forms (21
 * instructions instead of 16). s = tab[k % 32] + (ki << 47) is a 64-bit
 * shift and a 64-bit add (v_lshl_add_u64 itself only shifts by 0..4). tab
 * must point into LDS. */
__device__ static inline __attribute__((always_inline)) float kvexp_expf_core_fast(float x, const uint64_t *tab) {
    double xd, kd, r;
    const double c = KVEXP_EXP_INVLN2N, sh = KVEXP_EXP_SHIFT, nsh = -KVEXP_EXP_SHIFT;
    asm("v_cvt_f64_f32 %0, %3\n\t"
        "v_fma_f64 %1, %4, %0, %5\n\t"
        "v_add_f64 %2, %1, %6\n\t"
        "v_fma_f64 %2, %4, %0, -%2"
        : "=&v"(xd), "=&v"(kd), "=&v"(r)
        : "v"(x), "s"(c), "v"(sh), "s"(nsh));
    const uint64_t tb = tab[(uint32_t)kvexp_f64_bits(kd) & 31u];
    const double c0 = KVEXP_EXP_C0, c1 = KVEXP_EXP_C1, c2 = KVEXP_EXP_C2;
    double s, r2, p, y;
    float yf;
    asm("v_lshlrev_b64 %0, 47, %5\n\t"
        "v_lshl_add_u64 %0, %0, 0, %6\n\t"
        "v_mul_f64 %1, %7, %7\n\t"
        "v_fma_f64 %2, %8, %7, %9\n\t"
        "v_fma_f64 %3, %10, %7, 1.0\n\t"
        "v_fma_f64 %3, %2, %1, %3\n\t"
        "v_mul_f64 %3, %3, %0\n\t"
        "v_cvt_f32_f64 %4, %3"
        : "=&v"(s), "=&v"(r2), "=&v"(p), "=&v"(y), "=v"(yf)
        : "v"(kd), "v"(tb), "v"(r), "s"(c0), "v"(c1), "s"(c2));
    return yf;
}

/* kvexp_expf_core_fast in two halves, so that a caller evaluating several
 * exponentials can issue all their table reads before the first is needed:
 * kvexp_expf_reduce gives kd (the table index in the low bits of its bit
 * pattern) and r; kvexp_expf_finish takes them and the table entry
 * tb = tab[bits(kd) & 31]. The same operations in the same order. */
__device__ static inline __attribute__((always_inline)) void kvexp_expf_reduce(float x, double &kd, double &r) {
    double xd;
    const double c = KVEXP_EXP_INVLN2N, sh = KVEXP_EXP_SHIFT, nsh = -KVEXP_EXP_SHIFT;
    asm("v_cvt_f64_f32 %0, %3\n\t"
        "v_fma_f64 %1, %4, %0, %5\n\t"
        "v_add_f64 %2, %1, %6\n\t"
        "v_fma_f64 %2, %4, %0, -%2"
        : "=&v"(xd), "=&v"(kd), "=&v"(r)
        : "v"(x), "s"(c), "v"(sh), "s"(nsh));
}
__device__ static inline __attribute__((always_inline)) float kvexp_expf_finish(double kd, double r, uint64_t tb) {
    const double c0 = KVEXP_EXP_C0, c1 = KVEXP_EXP_C1, c2 = KVEXP_EXP_C2;
    double s, r2, p, y;
    float yf;
    asm("v_lshlrev_b64 %0, 47, %5\n\t"
        "v_lshl_add_u64 %0, %0, 0, %6\n\t"
        "v_mul_f64 %1, %7, %7\n\t"
        "v_fma_f64 %2, %8, %7, %9\n\t"
        "v_fma_f64 %3, %10, %7, 1.0\n\t"
        "v_fma_f64 %3, %2, %1, %3\n\t"
        "v_mul_f64 %3, %3, %0\n\t"
        "v_cvt_f32_f64 %4, %3"
        : "=&v"(s), "=&v"(r2), "=&v"(p), "=&v"(y), "=v"(yf)
        : "v"(kd), "v"(tb), "v"(r), "s"(c0), "v"(c1), "s"(c2));
    return yf;
}
#else
#define kvexp_expf_core_fast kvexp_expf_core_tab
#if defined(__HIPCC__)
/* Portable forms of the two halves (host pass; other expf forms). */
__device__ static inline void kvexp_expf_reduce(float x, double &kd, double &r) {
    const double xd = (double)x;
    kd = KVEXP_FMA64(KVEXP_EXP_INVLN2N, xd, KVEXP_EXP_SHIFT);
    r = KVEXP_FMA64(KVEXP_EXP_INVLN2N, xd, -(kd - KVEXP_EXP_SHIFT));
}
__device__ static inline float kvexp_expf_finish(double kd, double r, uint64_t tb) {
    const double s = kvexp_f64_from(tb + (kvexp_f64_bits(kd) << 47));
    const double p = KVEXP_FMA64(KVEXP_EXP_C0, r, KVEXP_EXP_C1);
    double y = KVEXP_FMA64(KVEXP_EXP_C2, r, 1.0);
    y = KVEXP_FMA64(p, r * r, y);
    return (float)(y * s);
}
#endif
#endif

/* kvexp_expf_tab_nb for arguments that are not positive (x <= 0, -0, -inf)
 * or NaN, as every softmax exponent is (s - m and m_prev - m with m the
 * running maximum); +0 is also handled. One special case remains:
 * x < -0x1.9fe368p6 (including -inf) -> +0. A NaN argument needs no case of
 * its own: it makes r NaN, so the polynomial and the result are NaN (the
 * payload may differ from glibc's x + x; every NaN is treated alike). */
KVEXP_HD float kvexp_expf_nonpos_nb(float x, const uint64_t *tab) {
    const float core = kvexp_expf_core_fast(x, tab);
    return x < -0x1.9fe368p6f ? 0.0f : core;
}

/* The reduction and polynomial with the built-in table. */
KVEXP_HD float kvexp_expf_core(float x) { return kvexp_expf_core_tab(x, kvexp_exp2_32_table); }

KVEXP_HD float kvexp_expf(float x) { return kvexp_expf_tab(x, kvexp_exp2_32_table); }

#endif /* KVEXP_EXPF_H */
