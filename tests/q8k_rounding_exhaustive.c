/* Exhaustive check of the Q8_K code formula the device quantizer uses
 * (q8k_code, swarmllm_amd/csrc/qmm_device.h) against the reference's steps
 * (BlockQ8K::from_float, k_quants.rs:2917-2920: t.round() half away from zero,
 * .min(127.) giving 127 for NaN, `as i8` saturating), for every one of the
 * 2^32 float bit patterns. Prints the number of mismatches; exit status 1 if
 * any. Built and run by tests/test_q8k_rounding.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static int reference(float t) {
    float r = roundf(t);
    float m = (r != r) ? 127.0f : (r < 127.0f ? r : 127.0f);
    if (m <= -128.0f) return -128;
    if (m >= 127.0f) return 127;
    return (int)m;
}

static int device_formula(float t) {
    volatile float h = copysignf(0.49999997f, t);
    volatile float s = t + h;                     /* one IEEE add, round to nearest even */
    float c = fmaxf(fminf(s, 127.49f), -128.49f); /* fminf first: NaN -> 127.49 */
    return (int)c;                                /* truncation, as v_cvt_i32_f32 */
}

int main(void) {
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t hi = 0; hi < 65536; hi++) {
        for (uint32_t lo = 0; lo < 65536; lo++) {
            const uint32_t b = ((uint32_t)hi << 16) | lo;
            float t;
            memcpy(&t, &b, 4);
            if (reference(t) != device_formula(t)) bad++;
        }
    }
    printf("%llu mismatches over 2^32 floats\n", (unsigned long long)bad);
    return bad != 0;
}
