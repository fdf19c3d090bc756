// Host check of chelis::erfcf_fast against CORE-MATH erfcf (test only):
// every binary32 input; where the fast path does not flag its result, the
// result must equal CORE-MATH's bit for bit. Prints the number of flagged
// inputs and of mismatches; exits nonzero on a mismatch.
#include <cstdio>
#include "../../chelis_amd/csrc/devmath.h"

extern "C" float chelis_crmath_ffi_erfcf(float);

int main() {
    long long mismatches = 0, flagged = 0;
#pragma omp parallel for reduction(+ : mismatches, flagged) schedule(dynamic, 1 << 16)
    for (long long i = 0; i < (1LL << 32); ++i) {
        const uint32_t bits = (uint32_t)i;
        const float x = chelis::f32_from(bits);
        bool slow;
        const float y = chelis::erfcf_fast(x, slow);
        if (slow) {
            ++flagged;
            continue;
        }
        const uint32_t want = chelis::f32_bits(chelis_crmath_ffi_erfcf(x));
        if (chelis::f32_bits(y) != want) {
            ++mismatches;
            if (mismatches < 8) std::printf("mismatch x=%08x got=%08x want=%08x\n", bits, chelis::f32_bits(y), want);
        }
    }
    std::printf("flagged %lld mismatches %lld\n", flagged, mismatches);
    return mismatches != 0;
}
