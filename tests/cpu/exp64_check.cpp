// Host check of the binary64 exp of devmath.h against CORE-MATH (test only).
// Usage: exp64_check N SEED FIXTURE...
//  - N seeded random inputs from five distributions, each through exp_cr (fast
//    path, else the fixed-point path) and through the fixed-point path alone
//    (exp_cr_slow), both compared with chelis_crmath_ffi_exp bit for bit;
//  - on the fast range, the fast path's double-double against the 128-bit
//    fixed-point value: the largest absolute error seen on y in [0.99, 2.02),
//    printed as log2 (the rounding test assumes at most 2^-73.7), and how
//    often the rounding test sends an input to the slow path;
//  - every "exp f64" row of the fixture files (input bits, MPFR-derived
//    expected bits) through exp_cr and exp_cr_slow.
// Prints "mismatches M" and exits nonzero when M > 0.
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include "../../chelis_amd/csrc/devmath.h"

extern "C" double chelis_crmath_ffi_exp(double);

using namespace chelis;

static uint64_t splitmix(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static double unit53(uint64_t &s) { return (double)(splitmix(s) >> 11) * 0x1p-53; }

static double draw(uint64_t &s, int kind) {
    switch (kind) {
        case 0:  // the whole finite, non-saturated domain
            return -746.0 + 1457.0 * unit53(s);
        case 1: {  // log-uniform magnitudes 2^-60 .. 2^9.5, either sign
            const uint64_t r = splitmix(s);
            const int e = -60 + (int)((r >> 1) % 70);
            double x = ldexp(1.0 + unit53(s), e);
            if (x > 700.0) x = 700.0 * unit53(s);
            return (r & 1) ? -x : x;
        }
        case 2: {  // near k ln2/64: the smallest reduced arguments
            const int64_t k = -68800 + (int64_t)(splitmix(s) % 134300);
            const double off = ldexp(unit53(s) - 0.5, -20 - (int)(splitmix(s) % 40));
            return (double)k * 0x1.62e42fefa39efp-7 + off;
        }
        case 3:  // softmax arguments x - max
            return -40.0 * unit53(s);
        default:  // the subnormal and overflow edges
            return (splitmix(s) & 1) ? -745.2 + 37.0 * unit53(s) : 709.0 + 0.8 * unit53(s);
    }
}

static long long report(const char *what, double x, double got, double want, long long &bad) {
    if (f64_bits(got) != f64_bits(want)) {
        if (bad < 12)
            std::printf("%s mismatch x=%016" PRIx64 " got=%016" PRIx64 " want=%016" PRIx64 "\n", what, f64_bits(x),
                        f64_bits(got), f64_bits(want));
        ++bad;
    }
    return bad;
}

int main(int argc, char **argv) {
    const long long n = argc > 1 ? std::atoll(argv[1]) : 1000000;
    const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 0) : 1;
    long long bad = 0, slow_count = 0, fast_count = 0, k_skips = 0;
    double max_err = 0.0;
#pragma omp parallel for reduction(+ : bad, slow_count, fast_count, k_skips) reduction(max : max_err) \
    schedule(dynamic, 4096)
    for (long long i = 0; i < n; ++i) {
        uint64_t s = seed * 0x100000001b3ull + (uint64_t)i * 0x9e3779b97f4a7c15ull;
        const double x = draw(s, (int)(i % 5));
        const double want = chelis_crmath_ffi_exp(x);
        long long b = 0;
        report("exp_cr", x, exp_cr(x), want, b);
        report("exp_cr_slow", x, exp_cr_slow(x), want, b);
        bad += b;
        if (x > -708.0 && x < 709.0) {
            bool slow;
            exp_fast(x, Exp2TableConst{}, slow);
            slow_count += slow;
            ++fast_count;
            const ExpDD d = exp_dd(x, Exp2TableConst{});
            int m;
            const U128 y = exp_fx(x, m);
            if (m != d.m) {
                ++k_skips;  // the two paths reduced with neighbouring k: different scalings
            } else {
                const U128 diff = sub128(add128(fixed_scaled(d.yh, 126), fixed_scaled(d.yl, 126)), y);
                const bool neg = (int64_t)diff.hi < 0;
                const U128 mag = neg ? sub128(U128{0, 0}, diff) : diff;
                const double err = ldexp((double)mag.hi, 64 - 126) + ldexp((double)mag.lo, -126);
                if (err > max_err) max_err = err;
            }
        }
    }
    for (int f = 3; f < argc; ++f) {
        FILE *fp = std::fopen(argv[f], "r");
        if (!fp) {
            std::printf("cannot open %s\n", argv[f]);
            return 2;
        }
        char line[512];
        long long rows = 0;
        while (std::fgets(line, sizeof line, fp)) {
            char fn[16], width[16];
            uint64_t xin, xout;
            if (std::sscanf(line, "%15s %15s %" SCNx64 " %" SCNx64, fn, width, &xin, &xout) != 4) continue;
            if (std::strcmp(fn, "exp") != 0 || std::strcmp(width, "f64") != 0) continue;
            const double x = f64_from(xin), want = f64_from(xout);
            report("fixture exp_cr", x, canon(exp_cr(x)), want, bad);
            report("fixture exp_cr_slow", x, canon(exp_cr_slow(x)), want, bad);
            ++rows;
        }
        std::fclose(fp);
        std::printf("fixture %s: %lld exp f64 rows\n", argv[f], rows);
    }
    std::printf("random %lld fast-range %lld slow-flagged %lld (1 in %.0f) k-skips %lld max-fast-error 2^%.2f\n", n,
                fast_count, slow_count, slow_count ? (double)fast_count / slow_count : 0.0, k_skips,
                max_err > 0 ? std::log2(max_err) : -999.0);
    std::printf("mismatches %lld\n", bad);
    return bad != 0;
}
