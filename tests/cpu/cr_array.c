/* Host side of the exhaustive binary32 transcendental checks (test only):
 * CORE-MATH (through the reference's FFI wrappers, which canonicalize NaN)
 * over a run of consecutive binary32 bit patterns, compared bit for bit
 * with results produced on the device. */
#include <stdint.h>
#include <string.h>

float chelis_crmath_ffi_expf(float);
float chelis_crmath_ffi_logf(float);
float chelis_crmath_ffi_erfcf(float);
float chelis_crmath_ffi_tanhf(float);

static float cr_one(int op, float x) {
    switch (op) {
        case 0: return chelis_crmath_ffi_expf(x);
        case 1: return chelis_crmath_ffi_logf(x);
        case 2: return chelis_crmath_ffi_erfcf(x);
        default: return chelis_crmath_ffi_tanhf(x);
    }
}

/* op: 0 exp, 1 log, 2 erfc, 3 tanh. got[i] is the device result for the
 * input bits first + i. Returns the number of mismatches; the first `cap`
 * are stored as (input bits, expected bits, device bits). */
long cr_check_run(int op, uint32_t first, long n, const uint32_t *got, uint32_t *bad, long cap) {
    long count = 0;
#pragma omp parallel for schedule(static, 65536)
    for (long i = 0; i < n; ++i) {
        const uint32_t xb = first + (uint32_t)i;
        float x;
        memcpy(&x, &xb, 4);
        const float w = cr_one(op, x);
        uint32_t wb;
        memcpy(&wb, &w, 4);
        if (wb != got[i]) {
            long slot;
#pragma omp atomic capture
            slot = count++;
            if (slot < cap) {
                bad[3 * slot] = xb;
                bad[3 * slot + 1] = wb;
                bad[3 * slot + 2] = got[i];
            }
        }
    }
    return count;
}

/* Binary64: CORE-MATH exp over explicit input bit patterns in[i], compared
 * with the device results got[i]; the first `cap` mismatches are stored as
 * (input bits, expected bits, device bits). */
double chelis_crmath_ffi_exp(double);

long cr_check64(int op, const uint64_t *in, long n, const uint64_t *got, uint64_t *bad, long cap) {
    long count = 0;
    (void)op; /* 0 exp: the only binary64 leaf held to correct rounding */
#pragma omp parallel for schedule(static, 65536)
    for (long i = 0; i < n; ++i) {
        double x;
        memcpy(&x, &in[i], 8);
        const double w = chelis_crmath_ffi_exp(x);
        uint64_t wb;
        memcpy(&wb, &w, 8);
        if (wb != got[i]) {
            long slot;
#pragma omp atomic capture
            slot = count++;
            if (slot < cap) {
                bad[3 * slot] = in[i];
                bad[3 * slot + 1] = wb;
                bad[3 * slot + 2] = got[i];
            }
        }
    }
    return count;
}
