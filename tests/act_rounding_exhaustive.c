/* Exhaustive check of the code formulas the device activation quantizers use
 * (swarmllm_amd/csrc/qmm_device.h) against the reference's steps, for every
 * one of the 2^32 float bit patterns:
 *   q8k_code  vs BlockQ8K::from_float (k_quants.rs:2917-2920): t.round() half
 *             away from zero, .min(127.) giving 127 for NaN, `as i8`;
 *   q8_0_code vs BlockQ8_0::from_float (k_quants.rs:1262-1265): t.round(),
 *             `as i8` (saturating, NaN gives 0), with v_cvt_i32_f32 modelled
 *             as the ISA states it: truncation, saturation, NaN to 0.
 * Prints the number of mismatches; exit status 1 if any. Built and run by
 * tests/test_act_rounding.py. */
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

static int reference_q8_0(float t) {
    float r = roundf(t);
    if (r != r) return 0;
    if (r <= -128.0f) return -128;
    if (r >= 127.0f) return 127;
    return (int)r;
}

static int32_t cvt_i32_f32(float f) { /* v_cvt_i32_f32 */
    if (f != f) return 0;
    if (f >= 2147483648.0f) return 2147483647;
    if (f <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)f;
}

static int device_q8_0(float t) {
    volatile float h = copysignf(0.49999997f, t);
    volatile float s = t + h;
    int32_t q = cvt_i32_f32(s);
    return q < -128 ? -128 : (q > 127 ? 127 : q);
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
            if (reference_q8_0(t) != device_q8_0(t)) bad++;
        }
    }
    printf("%llu mismatches over 2^32 floats\n", (unsigned long long)bad);
    return bad != 0;
}
