// Host check of devmath.h's faithful binary64 exp for arguments <= 0 or NaN
// (the default binary64 softmax row) against CORE-MATH (test only).
// Usage: exp64_faithful_check N SEED
//  - N seeded arguments from four distributions (the whole nonpositive
//    range down to -750, softmax-like x - max, tiny magnitudes, the
//    subnormal edge), each compared with chelis_crmath_ffi_exp: on normal
//    results the error in ulps of the correctly rounded result, below
//    2^-1022 the error in units of the least subnormal;
//  - special arguments: +0 and -0 give exactly 1, -inf and -746 give +0,
//    NaN gives a NaN.
// Prints "max-ulp U max-subnormal-units S specials-bad B".
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include "../../chelis_amd/csrc/devmath.h"

extern "C" double chelis_crmath_ffi_exp(double);

using namespace chelis;

struct TabHi {
    double operator()(int j) const { return chelis_exp2_64_tab[j][0]; }
};

static uint64_t splitmix(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static double unit53(uint64_t &s) { return (double)(splitmix(s) >> 11) * 0x1p-53; }

static double draw(uint64_t &s, int kind) {
    switch (kind) {
        case 0: return -750.0 * unit53(s);
        case 1: return -40.0 * unit53(s);
        case 2: return -ldexp(1.0 + unit53(s), -60 + (int)(splitmix(s) % 66));
        default: return -745.2 + 40.0 * unit53(s);
    }
}

int main(int argc, char **argv) {
    const long long n = argc > 1 ? std::atoll(argv[1]) : 1000000;
    const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 0) : 1;
    double max_ulp = 0.0, max_sub = 0.0;
#pragma omp parallel for reduction(max : max_ulp, max_sub) schedule(dynamic, 4096)
    for (long long i = 0; i < n; ++i) {
        uint64_t s = seed * 0x100000001b3ull + (uint64_t)i * 0x9e3779b97f4a7c15ull;
        const double x = draw(s, (int)(i % 4));
        const double want = chelis_crmath_ffi_exp(x);
        const double got = exp_nonpos_faithful(x, TabHi{});
        if (want >= 0x1p-1022) {
            const double u = std::fabs(got - want) / ldexp(1.0, std::ilogb(want) - 52);
            if (u > max_ulp) max_ulp = u;
        } else {
            const double u = std::fabs(got - want) / 0x1p-1074;
            if (u > max_sub) max_sub = u;
        }
    }
    int bad = 0;
    bad += f64_bits(exp_nonpos_faithful(0.0, TabHi{})) != f64_bits(1.0);
    bad += f64_bits(exp_nonpos_faithful(-0.0, TabHi{})) != f64_bits(1.0);
    bad += f64_bits(exp_nonpos_faithful(-INFINITY, TabHi{})) != 0;
    bad += f64_bits(exp_nonpos_faithful(-746.0, TabHi{})) != 0;
    bad += !std::isnan(exp_nonpos_faithful(NAN, TabHi{}));
    bad += !std::isnan(exp_nonpos_faithful(-NAN, TabHi{}));
    std::printf("checked %lld max-ulp %.4f max-subnormal-units %.4f specials-bad %d\n", n, max_ulp, max_sub, bad);
    return bad ? 1 : 0;
}
