// Host check of chelis::expf_cr and chelis::expf_cr_nonpos against the
// CORE-MATH oracle (test only).
// Usage: expf_check STRIDE  -> checks every STRIDE-th binary32 bit pattern,
// prints the number of mismatching results and the first few inputs.
#include <cstdio>
#include <cstdlib>
#include "../../chelis_amd/csrc/devmath.h"

extern "C" float chelis_crmath_ffi_expf(float);

int main(int argc, char **argv) {
    const long long stride = argc > 1 ? std::atoll(argv[1]) : 1;
    const long long count = (1LL << 32) / stride;
    long long mismatches = 0;
#pragma omp parallel for reduction(+ : mismatches) schedule(dynamic, 1 << 16)
    for (long long i = 0; i < count; ++i) {
        uint32_t bits = (uint32_t)(i * stride);
        float x = chelis::f32_from(bits);
        uint32_t got = chelis::f32_bits(chelis::expf_cr(x));
        uint32_t want = chelis::f32_bits(chelis_crmath_ffi_expf(x));
        if (got != want) {
            ++mismatches;
            if (mismatches < 8) std::printf("mismatch x=%08x got=%08x want=%08x\n", bits, got, want);
        }
        // the non-positive specialization: sign bit set, +0, positive NaNs
        if ((bits >> 31) || bits == 0u || (bits & 0x7fffffffu) > 0x7f800000u) {
            uint32_t got_np = chelis::f32_bits(chelis::expf_cr_nonpos(x));
            if (got_np != want) {
                ++mismatches;
                if (mismatches < 8) std::printf("nonpos mismatch x=%08x got=%08x want=%08x\n", bits, got_np, want);
            }
        }
    }
    std::printf("checked %lld mismatches %lld\n", count, mismatches);
    return mismatches != 0;
}
