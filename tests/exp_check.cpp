// Compares the exp restatement of silvic_amd/csrc/exp_f64.hpp (host build) with the C library's exp, bit for
// bit, on random inputs over the ranges the binary gradients see and on special values. Prints the mismatches.
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "../silvic_amd/csrc/exp_f64.hpp"

int main(int argc, char **argv) {
    long n = argc > 1 ? atol(argv[1]) : 1000000;
    uint64_t s = 88172645463325252ull;
    long bad = 0;
    for (long i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        double u = static_cast<double>(s >> 11) / 9007199254740992.0;
        double x;
        switch (i % 4) {
        case 0: x = u * 60 - 30; break;                                   // gradient range
        case 1: x = static_cast<double>(static_cast<float>(u * 40 - 20)); break;  // f32 scores
        case 2: x = u * 2100 - 1050; break;                               // over/underflow ranges
        default: x = (u - 0.5) * 1e-12; break;                            // near zero
        }
        double a = std::exp(x), b = srocm_exp::exp(x);
        if (srocm_exp::asu(a) != srocm_exp::asu(b)) ++bad;
    }
    const double special[] = {0.0, -0.0, 1e-300, -1e-300, 709.78, 709.79, -745.1, -745.2, 1e6, -1e6, INFINITY,
                              -INFINITY, 511.9, 512.0, -512.0, -700.5, -708.4, 600.25, 0x1p-54, -0x1p-55};
    for (double x : special)
        if (srocm_exp::asu(std::exp(x)) != srocm_exp::asu(srocm_exp::exp(x))) ++bad;
    if (!std::isnan(srocm_exp::exp(NAN))) ++bad;
    printf("%ld\n", bad);
    return 0;
}
