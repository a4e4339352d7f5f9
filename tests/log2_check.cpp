// The double-double log2 bracket of silvic_amd/csrc/log2_dd.hpp, built for the host with -ffp-contract=off as the
// device build is.
//   log2_check glibc N SEED : N pseudo-random x = 1 + s (s spread over 2^-60 .. 2^40, plus powers of two and values
//                             next to them); prints the number of x whose C-library log2 is not the bracket's
//                             (outside {lo, hi}, or not lo when the value is a double), the undecided ones, and N
//   log2_check dump         : reads x values (hex floats) from stdin, prints "x lo hi status" in hex per line
//   log2_check table        : prints the number of entries of the reciprocal table that differ from dd_recip's
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../silvic_amd/csrc/log2_dd.hpp"

static uint64_t rng = 0;
static uint64_t next_u64() {  // splitmix64
    uint64_t z = (rng += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int main(int argc, char **argv) {
    if (argc >= 4 && !strcmp(argv[1], "glibc")) {
        const long n = atol(argv[2]);
        rng = strtoull(argv[3], nullptr, 10);
        long bad = 0, undecided = 0;
        for (long i = 0; i < n; ++i) {
            double x;
            const uint64_t r = next_u64();
            if (i % 16 == 0) {  // a power of two, or one of its neighbours
                const double p = std::ldexp(1.0, static_cast<int>(r % 80));
                const int w = static_cast<int>((r >> 8) % 3);
                x = w == 0 ? p : (w == 1 ? std::nextafter(p, 0.0) : std::nextafter(p, INFINITY));
                if (x < 1.0) x = 1.0;
            } else {
                const double u = static_cast<double>(r >> 11) * 0x1p-53;      // [0, 1)
                const double s = std::exp2(-60.0 + 100.0 * u);                 // 2^-60 .. 2^40
                x = 1.0 + s;
            }
            double lo, hi;
            const int st = srocm_log2::log2_bracket(x, lo, hi);
            const double c = std::log2(x);
            if (st == 2) {
                ++undecided;
                continue;
            }
            if (st == 0 ? c != lo : (c != lo && c != hi)) ++bad;
        }
        printf("%ld %ld %ld\n", bad, undecided, n);
        return 0;
    }
    if (argc >= 2 && !strcmp(argv[1], "table")) {  // the reciprocal table against dd_recip's fma residuals
        int bad = 0;
        for (int k = 0; k < 22; ++k) {
            const srocm_log2::DD r = srocm_log2::dd_recip(2.0 * k + 1.0);
            bad += r.hi != srocm_log2::RECIP[k][0] || r.lo != srocm_log2::RECIP[k][1];
        }
        printf("%d\n", bad);
        return 0;
    }
    if (argc >= 2 && !strcmp(argv[1], "dump")) {
        char buf[128];
        while (scanf("%127s", buf) == 1) {
            const double x = strtod(buf, nullptr);
            double lo, hi;
            const int st = srocm_log2::log2_bracket(x, lo, hi);
            printf("%a %a %a %d\n", x, lo, hi, st);
        }
        return 0;
    }
    fprintf(stderr, "usage: log2_check glibc N SEED | log2_check dump\n");
    return 2;
}
