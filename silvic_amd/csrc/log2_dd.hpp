// log2_dd.hpp - the two doubles that bracket log2(x), from log2(x) evaluated in double-double arithmetic, for the
// lambdarank normalization factor log2(1 + s) / s (objective/lambdarank.rs:322-326) made on the device.
//
// The C library's log2 is within one ulp of the exact value (glibc documents at most 1 ulp on x86-64; its
// table-driven log2 is bounded at 0.55 ulp), so whatever it returns is one of the two doubles around the exact
// value: round-down or round-up. Each candidate factor gives the row's f32 gradient; where both give the same f32
// for every row of a query, the device's result is the host's whatever the host's log2 returned, and otherwise the
// query is left to the host.
//
// The method: x = 2^e m with m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh t with t = (m - 1) / (m + 1), |t| < 0.1716,
// and atanh t = t (1 + t^2/3 + t^4/5 + ...), 22 terms evaluated by Horner's rule in double-double (each term below
// 2^-107 of the sum beyond them), then log2 x = e + ln m / ln 2 with 1/ln 2 as a double-double constant. Every
// double-double operation is exact to about 2^-104 relative, so the result is within 2^-98 of log2 x relative; a
// value closer than 2^-95 to a double is reported as undecided. Build with -ffp-contract=off: the error-free
// transformations need each product and sum rounded on its own.
#pragma once

#include <stdint.h>
#include <string.h>

#include <cmath>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define SROCM_LOG2_HD __host__ __device__
#else
#define SROCM_LOG2_HD
#endif

namespace srocm_log2 {

struct DD {
    double hi, lo;
};

SROCM_LOG2_HD inline double fma_(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_fma(a, b, c);
#else
    return std::fma(a, b, c);
#endif
}

SROCM_LOG2_HD inline DD two_sum(double a, double b) {
    const double s = a + b;
    const double bb = s - a;
    return DD{s, (a - (s - bb)) + (b - bb)};
}
SROCM_LOG2_HD inline DD quick_two_sum(double a, double b) {  // |a| >= |b|
    const double s = a + b;
    return DD{s, b - (s - a)};
}
SROCM_LOG2_HD inline DD dd_add(DD a, DD b) {
    DD s = two_sum(a.hi, b.hi);
    const DD t = two_sum(a.lo, b.lo);
    s.lo += t.hi;
    s = quick_two_sum(s.hi, s.lo);
    s.lo += t.lo;
    return quick_two_sum(s.hi, s.lo);
}
SROCM_LOG2_HD inline DD dd_mul(DD a, DD b) {
    const double p = a.hi * b.hi;
    double e = fma_(a.hi, b.hi, -p);
    e += a.hi * b.lo + a.lo * b.hi;
    return quick_two_sum(p, e);
}
// 1 / k as a double-double for a small positive integer k: the residual 1 - hi k is exact by fma
SROCM_LOG2_HD inline DD dd_recip(double k) {
    const double hi = 1.0 / k;
    return DD{hi, fma_(-hi, k, 1.0) / k};
}

SROCM_LOG2_HD inline uint64_t bits(double x) {
    uint64_t u;
    memcpy(&u, &x, 8);
    return u;
}
SROCM_LOG2_HD inline double from_bits(uint64_t u) {
    double x;
    memcpy(&x, &u, 8);
    return x;
}

// 1 / (2k + 1), k = 0..21, as double-doubles: the double nearest each and the double nearest the rest (computed in
// 60-digit decimal arithmetic; dd_recip makes the same pairs with an fma)
constexpr double RECIP[22][2] = {
    {0x1.0000000000000p+0, 0x0.0p+0},  // 1/1
    {0x1.5555555555555p-2, 0x1.5555555555555p-56},  // 1/3
    {0x1.999999999999ap-3, -0x1.999999999999ap-57},  // 1/5
    {0x1.2492492492492p-3, 0x1.2492492492492p-57},  // 1/7
    {0x1.c71c71c71c71cp-4, 0x1.c71c71c71c71cp-58},  // 1/9
    {0x1.745d1745d1746p-4, -0x1.745d1745d1746p-59},  // 1/11
    {0x1.3b13b13b13b14p-4, -0x1.3b13b13b13b14p-58},  // 1/13
    {0x1.1111111111111p-4, 0x1.1111111111111p-60},  // 1/15
    {0x1.e1e1e1e1e1e1ep-5, 0x1.e1e1e1e1e1e1ep-61},  // 1/17
    {0x1.af286bca1af28p-5, 0x1.af286bca1af28p-59},  // 1/19
    {0x1.8618618618618p-5, 0x1.8618618618618p-59},  // 1/21
    {0x1.642c8590b2164p-5, 0x1.642c8590b2164p-60},  // 1/23
    {0x1.47ae147ae147bp-5, -0x1.eb851eb851eb8p-61},  // 1/25
    {0x1.2f684bda12f68p-5, 0x1.2f684bda12f68p-59},  // 1/27
    {0x1.1a7b9611a7b96p-5, 0x1.1a7b9611a7b96p-61},  // 1/29
    {0x1.0842108421084p-5, 0x1.0842108421084p-60},  // 1/31
    {0x1.f07c1f07c1f08p-6, -0x1.f07c1f07c1f08p-61},  // 1/33
    {0x1.d41d41d41d41dp-6, 0x1.0750750750750p-60},  // 1/35
    {0x1.bacf914c1bad0p-6, -0x1.bacf914c1bad0p-60},  // 1/37
    {0x1.a41a41a41a41ap-6, 0x1.0690690690690p-60},  // 1/39
    {0x1.8f9c18f9c18fap-6, -0x1.f3831f3831f38p-61},  // 1/41
    {0x1.7d05f417d05f4p-6, 0x1.7d05f417d05f4p-62},  // 1/43
};

// 1 / ln 2 = 1.442695040888963407359924681001892137...: the double nearest it and the double nearest the rest
constexpr double INV_LN2_HI = 0x1.71547652b82fep+0;
constexpr double INV_LN2_LO = 0x1.777d0ffda0d24p-56;
constexpr double SQRT_HALF = 0x1.6a09e667f3bcdp-1;

// log2 x for a finite x >= 1 (the factor's 1 + s), as a normalized double-double.
SROCM_LOG2_HD inline DD log2_dd(double x) {
    int e = 0;
    double m = __builtin_frexp(x, &e);  // x = m 2^e, m in [0.5, 1)
    if (m < SQRT_HALF) {
        m *= 2.0;
        e -= 1;
    }
    const double num = m - 1.0;              // exact: m lies in [0.5, 2]
    const DD den = two_sum(m, 1.0);          // m + 1, exactly
    const double t_hi = num / den.hi;
    double r = fma_(-t_hi, den.hi, num);     // the division's residual, exact
    r -= t_hi * den.lo;
    const DD t{t_hi, r / den.hi};
    const DD u = dd_mul(t, t);
    // S = sum_{k=0}^{21} u^k / (2k + 1) by Horner's rule
    DD s{RECIP[21][0], RECIP[21][1]};
    for (int k = 20; k >= 0; --k) s = dd_add(dd_mul(s, u), DD{RECIP[k][0], RECIP[k][1]});
    DD ln_m = dd_mul(t, s);
    ln_m.hi *= 2.0;
    ln_m.lo *= 2.0;
    const DD l2 = dd_mul(ln_m, DD{INV_LN2_HI, INV_LN2_LO});
    return dd_add(DD{static_cast<double>(e), 0.0}, l2);
}

// The doubles just below and just above log2 x (x finite, x >= 1): returns 0 when log2 x is a double (lo = hi =
// it), 1 when lo < log2 x < hi are its neighbours, 2 when the evaluation cannot tell on which side of a double the
// value lies.
SROCM_LOG2_HD inline int log2_bracket(double x, double &lo, double &hi) {
    const DD y = log2_dd(x);
    if (y.lo == 0.0) {
        lo = hi = y.hi;
        return y.hi == __builtin_floor(y.hi) ? 0 : 2;  // only powers of two have a double logarithm
    }
    if (__builtin_fabs(y.lo) < 0x1p-95 * __builtin_fabs(y.hi)) {
        lo = hi = y.hi;
        return 2;
    }
    // y.hi > 0 here (x > 1): neighbours are one unit of the bit pattern away
    if (y.lo > 0.0) {
        lo = y.hi;
        hi = from_bits(bits(y.hi) + 1u);
    } else {
        lo = from_bits(bits(y.hi) - 1u);
        hi = y.hi;
    }
    return 1;
}

}  // namespace srocm_log2
