// Host check of chelis::quot_f32 (binary32 v / t through a binary64
// reciprocal) against IEEE binary32 division (test only).
// Every binary32 v in [2^-149, 1] against a set of totals t, plus random
// (v, t) pairs; prints the number of mismatches.
#include <cstdio>
#include <cstdlib>
#include "../../chelis_amd/csrc/devmath.h"

int main(int argc, char **argv) {
    const long long stride = argc > 1 ? std::atoll(argv[1]) : 1;
    const float totals[] = {1.0f, 1.5f, 3.0f, 7.0f, 10.0f, 1023.75f, 1024.0f, 4096.0f, 1.1f, 2.7182817f,
                            123.456f, 16777215.0f, 0x1.fffffep+0f, 0x1.000002p+0f, 97.0f, 4097.0f};
    long long mismatches = 0, checked = 0;
    for (float t : totals) {
        const double inv = 1.0 / (double)t;
        const long long hi = (long long)chelis::f32_bits(1.0f);
#pragma omp parallel for reduction(+ : mismatches, checked) schedule(dynamic, 1 << 16)
        for (long long b = 1; b <= hi; b += stride) {
            const float v = chelis::f32_from((uint32_t)b);
            ++checked;
            if (chelis::f32_bits(chelis::quot_f32(v, inv)) != chelis::f32_bits(v / t)) ++mismatches;
        }
    }
    // random pairs: t in [1, 2^24), v in [0, 1]
    unsigned long long s = 0x9E3779B97F4A7C15ull;
    for (long long i = 0; i < (1LL << 26); ++i) {
        s ^= s << 13, s ^= s >> 7, s ^= s << 17;
        const float t = 1.0f + (float)((s >> 40) & 0xffffff);
        const float v = chelis::f32_from((uint32_t)(s & 0x3f800000u) | (uint32_t)((s >> 8) & 0x7fffff));
        ++checked;
        if (chelis::f32_bits(chelis::quot_f32(v, 1.0 / (double)t)) != chelis::f32_bits(v / t)) ++mismatches;
    }
    std::printf("checked %lld mismatches %lld\n", checked, mismatches);
    return mismatches != 0;
}
