// exp_f64.hpp - double-precision exp, bit-identical to the C library's on the hosts silvic's CPU trainer runs on
// (glibc >= 2.28 on x86-64 with FMA), for the binary-logloss gradients (objective/binary.rs:43).
//
// The method is the table-driven exp of ARM optimized-routines (Szabolcs Nagy), which glibc ships as its exp:
// exp(x) = 2^(k/N) * exp(r) with N = 128, x = k ln2/N + r, |r| <= ln2/(2N); 2^(k/N) from a 128-entry table
// (exp_table.h, generated from exact arithmetic) and exp(r) - 1 ~= r + C2 r^2 + C3 r^3 + C4 r^4 + C5 r^5 with the
// published minimax coefficients. glibc's x86-64 build compiles it with fused multiply-adds wherever a product
// feeds one addition; the same five fmas are written out here, everything else is plain IEEE arithmetic
// (build with -ffp-contract=off). Inputs with |x| >= 512 take the published special-case path.
#pragma once

#include <stdint.h>
#include <string.h>

#include <cmath>

#include "exp_table.h"

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define SROCM_HD __host__ __device__
#else
#define SROCM_HD
#endif

namespace srocm_exp {

#ifdef __HIPCC__
__constant__ const uint64_t TAB_D[256] = {SROCM_EXP_TABLE_DATA};
#endif
static const uint64_t TAB_H[256] = {SROCM_EXP_TABLE_DATA};

SROCM_HD inline uint64_t asu(double x) {
    uint64_t u;
    memcpy(&u, &x, 8);
    return u;
}
SROCM_HD inline double asd(uint64_t u) {
    double x;
    memcpy(&x, &u, 8);
    return x;
}
SROCM_HD inline uint64_t tab(uint64_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return TAB_D[i];
#else
    return TAB_H[i];
#endif
}
SROCM_HD inline double fused(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_fma(a, b, c);
#else
    return std::fma(a, b, c);
#endif
}

constexpr double INV_LN2_N = 0x1.71547652b82fep0 * 128;
constexpr double NEG_LN2_HI_N = -0x1.62e42fefa0000p-8;
constexpr double NEG_LN2_LO_N = -0x1.cf79abc9e3b3ap-47;
constexpr double SHIFT = 0x1.8p52;
constexpr double C2 = 0x1.ffffffffffdbdp-2;
constexpr double C3 = 0x1.555555555543cp-3;
constexpr double C4 = 0x1.55555cf172b91p-5;
constexpr double C5 = 0x1.1111167a4d017p-7;

// |x| in [512, 1024): the scale's exponent may over- or underflow; rescale around it.
SROCM_HD inline double special_case(double tmp, uint64_t sbits, uint64_t ki) {
    if ((ki & 0x80000000ull) == 0) {
        sbits -= 1009ull << 52;
        double scale = asd(sbits);
        return 0x1p1009 * fused(scale, tmp, scale);
    }
    // the product feeds two sums here, so it is rounded once and not fused
    sbits += 1022ull << 52;
    double scale = asd(sbits);
    double p = scale * tmp;
    double y = scale + p;
    if (y < 1.0) {
        double lo = scale - y + p;
        double hi = 1.0 + y;
        lo = 1.0 - hi + y + lo;
        y = (hi + lo) - 1.0;
        if (y == 0.0) y = 0.0;
    }
    return 0x1p-1022 * y;
}

SROCM_HD inline double exp(double x) {
    uint32_t abstop = static_cast<uint32_t>(asu(x) >> 52) & 0x7ffu;
    if (abstop - 0x3c9u >= 0x408u - 0x3c9u) {  // |x| < 2^-54, or |x| >= 512, or NaN/inf
        if (abstop - 0x3c9u >= 0x80000000u) return 1.0 + x;
        if (abstop >= 0x409u) {                  // |x| >= 1024
            if (asu(x) == 0xfff0000000000000ull) return 0.0;
            if (abstop >= 0x7ffu) return 1.0 + x;
            return (asu(x) >> 63) ? 0.0 : asd(0x7ff0000000000000ull);
        }
        abstop = 0;
    }
    double kd = fused(INV_LN2_N, x, SHIFT);
    uint64_t ki = asu(kd);
    kd -= SHIFT;
    double r = fused(kd, NEG_LN2_LO_N, fused(kd, NEG_LN2_HI_N, x));
    uint64_t idx = 2 * (ki % 128);
    uint64_t top = ki << 45;
    double tail = asd(tab(idx));
    uint64_t sbits = tab(idx + 1) + top;
    double r2 = r * r;
    double tmp = fused(r2 * r2, fused(r, C5, C4), fused(r2, fused(r, C3, C2), tail + r));
    if (abstop == 0) return special_case(tmp, sbits, ki);
    double scale = asd(sbits);
    return fused(scale, tmp, scale);
}

}  // namespace srocm_exp
