/*
 * qref_formats.c — block formats of the reference's quantized path:
 * f16 conversion, weight/activation quantizers (from_float), dequantizers
 * (to_float) and the scalar dot products (vec_dot_unopt).
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + CPU baseline), see qref.h.
 * Every function cites the reference lines it restates; paths are relative
 * to vendor/candle/candle-core/src/quantized/ in the reference checkout.
 */
#include "qref.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

_Static_assert(sizeof(qref_q4_0) == 18, "q4_0");
_Static_assert(sizeof(qref_q8_0) == 34, "q8_0");
_Static_assert(sizeof(qref_q4_k) == 144, "q4_k");
_Static_assert(sizeof(qref_q6_k) == 210, "q6_k");
_Static_assert(sizeof(qref_q8_k) == 292, "q8_k");
_Static_assert(sizeof(qref_mxfp4) == 17, "mxfp4");
_Static_assert(sizeof(qref_iq4_nl) == 18, "iq4_nl");

/* ---------------------------------------------------------------------- */
/* registry: Q/mod.rs:294-461                                              */
/* ---------------------------------------------------------------------- */
int qref_block_size(int type) {
    switch (type) {
    case QREF_Q4_0: case QREF_Q8_0: case QREF_MXFP4: case QREF_IQ4_NL: return 32;
    case QREF_Q4_K: case QREF_Q6_K: case QREF_Q8_K: return 256;
    default: return 0;
    }
}

int qref_type_size(int type) {
    switch (type) {
    case QREF_Q4_0: return 18;
    case QREF_Q8_0: return 34;
    case QREF_Q4_K: return 144;
    case QREF_Q6_K: return 210;
    case QREF_Q8_K: return 292;
    case QREF_MXFP4: return 17;
    case QREF_IQ4_NL: return 18;
    default: return 0;
    }
}

/* VecDotType: Q/k_quants.rs:322 (Q4_0), :462 (MXFP4), :706 (IQ4_NL),
 * :1219 (Q8_0), :2006 (Q4_K), :2573 (Q6_K). */
int qref_vec_dot_type(int type) {
    switch (type) {
    case QREF_Q4_0: case QREF_Q8_0: case QREF_MXFP4: case QREF_IQ4_NL: return QREF_Q8_0;
    case QREF_Q4_K: case QREF_Q6_K: case QREF_Q8_K: return QREF_Q8_K;
    default: return 0;
    }
}

/* ---------------------------------------------------------------------- */
/* f16 <-> f32, IEEE binary16 with round-to-nearest-even (half 2.7.1).      */
/* Pinned by tests against numpy.float16 (an independent IEEE RNE routine). */
/* ---------------------------------------------------------------------- */
uint16_t qref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e8 = (x >> 23) & 0xFFu;
    const uint32_t m23 = x & 0x7FFFFFu;
    if (e8 == 0xFFu) { /* inf or nan: a nan keeps its top payload bits, quiet */
        return (uint16_t)(sign | 0x7C00u | (m23 ? (0x200u | (m23 >> 13)) : 0u));
    }
    const int e = (int)e8 - 127 + 15; /* biased half exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) { /* subnormal half (or zero) */
        if (e < -10) return (uint16_t)sign;
        const uint32_t m = m23 | 0x800000u;   /* 24 significant bits */
        const int shift = 14 - e;             /* 14..24 */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (m23 >> 13);
    const uint32_t rem = m23 & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry into the exponent: correct */
    return (uint16_t)(sign | h);
}

float qref_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0x1Fu) {
        x = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else { /* subnormal half: normalise */
        int ee = -14;
        while ((m & 0x400u) == 0) { m <<= 1; ee--; }
        m &= 0x3FFu;
        x = sign | ((uint32_t)(ee + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---------------------------------------------------------------------- */
/* Rust numeric semantics                                                   */
/* ---------------------------------------------------------------------- */
/* `f as i32` / `as i8` / `as u8`: truncate toward zero, saturate, NaN -> 0. */
static inline int32_t rs_as_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
static inline int8_t rs_as_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
static inline uint8_t rs_as_u8(float v) {
    if (v != v) return 0;
    if (v >= 255.0f) return 255;
    if (v <= 0.0f) return 0;
    return (uint8_t)v;
}
/* f32::max / f32::min: the non-NaN operand wins; between equal values
 * (including +0/-0) the second operand is returned. */
static inline float rs_max(float self, float other) {
    if (other != other) return self;
    if (self != self) return other;
    return self > other ? self : other;
}
static inline float rs_min(float self, float other) {
    if (other != other) return self;
    if (self != self) return other;
    return self < other ? self : other;
}
/* Q/utils.rs:1 `nearest_int`: f32::round (half away from zero), then `as i32`. */
static inline int32_t nearest_int(float v) { return rs_as_i32(roundf(v)); }
static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* f32::total_cmp key (core::f32::total_cmp). */
static inline int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

/* ---------------------------------------------------------------------- */
/* tables: Q/k_quants.rs:30-54                                              */
/* ---------------------------------------------------------------------- */
static const int8_t IQ4NL_VALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1, 13, 25, 38, 53, 69, 89, 113};
static const int8_t MXFP4_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* e8m0_half_bits: Q/k_quants.rs:39-46 (2^(e-128), subnormal for e < 2). */
static inline float e8m0_to_f32_half(uint8_t e) {
    const uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ---------------------------------------------------------------------- */
/* Q8_0: Q/k_quants.rs:1216-1313                                           */
/* ---------------------------------------------------------------------- */
/* from_float: Q/k_quants.rs:1240-1269 */
static void q8_0_from_float(const float *x, qref_q8_0 *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float *xs = x + 32 * i;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = rs_max(amax, fabsf(xs[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = qref_f32_to_f16(d);
        for (int j = 0; j < 32; j++) y[i].qs[j] = rs_as_i8(roundf(xs[j] * id));
    }
}
/* to_float: Q/k_quants.rs:1222-1238 */
static void q8_0_to_float(const qref_q8_0 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = qref_f16_to_f32(x[i].d);
        for (int j = 0; j < 32; j++) y[32 * i + j] = (float)x[i].qs[j] * d;
    }
}
/* vec_dot_unopt: Q/k_quants.rs:1294-1312 */
static float q8_0_dot_unopt(int64_t nb, const qref_q8_0 *x, const qref_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)x[i].qs[j] * (int32_t)y[i].qs[j];
        sumf += (float)s * qref_f16_to_f32(x[i].d) * qref_f16_to_f32(y[i].d);
    }
    return sumf;
}

/* ---------------------------------------------------------------------- */
/* Q4_0: Q/k_quants.rs:319-427 (kept to pin the driver with the reference's */
/* closed-form matmul vectors, tests/quantized_tests.rs:91-221)             */
/* ---------------------------------------------------------------------- */
/* from_float: Q/k_quants.rs:346-377 */
static void q4_0_from_float(const float *x, qref_q4_0 *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float *xs = x + 32 * i;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); max = xs[j]; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = qref_f32_to_f16(d);
        for (int j = 0; j < 16; j++) {
            const float x0 = xs[j] * id;
            const float x1 = xs[16 + j] * id;
            uint8_t xi0 = rs_as_u8(x0 + 8.5f);
            uint8_t xi1 = rs_as_u8(x1 + 8.5f);
            if (xi0 > 15) xi0 = 15;
            if (xi1 > 15) xi1 = 15;
            y[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}
/* to_float: Q/k_quants.rs:325-345 */
static void q4_0_to_float(const qref_q4_0 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = qref_f16_to_f32(x[i].d);
        for (int j = 0; j < 16; j++) {
            y[32 * i + j] = (float)((int)(x[i].qs[j] & 0x0F) - 8) * d;
            y[32 * i + j + 16] = (float)((int)(x[i].qs[j] >> 4) - 8) * d;
        }
    }
}
/* vec_dot_unopt: Q/k_quants.rs:409-426 */
static float q4_0_dot_unopt(int64_t nb, const qref_q4_0 *x, const qref_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        int32_t s = 0;
        for (int j = 0; j < 16; j++) {
            const int v0 = (int)(x[i].qs[j] & 0x0F) - 8;
            const int v1 = (int)(x[i].qs[j] >> 4) - 8;
            s += v0 * y[i].qs[j] + v1 * y[i].qs[j + 16];
        }
        sumf += (float)s * qref_f16_to_f32(x[i].d) * qref_f16_to_f32(y[i].d);
    }
    return sumf;
}

/* ---------------------------------------------------------------------- */
/* Q8_K: Q/k_quants.rs:2844-2941                                           */
/* ---------------------------------------------------------------------- */
/* q8k_scale(): Q/k_quants.rs:145-152 — 127 (llama.cpp), or candle's older
 * 128 under SWARMLLM_Q8K_SCALE=128 (the reference's A/B knob). */
static float g_q8k_scale = 127.0f;
void qref_set_q8k_scale(float s) { g_q8k_scale = s; }

/* from_float: Q/k_quants.rs:2882-2927. */
static void q8_k_from_float(const float *x, qref_q8_k *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float *xs = x + 256 * i;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); max = xs[j]; }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, 256);
            /* bsums are left as they were (the reference writes none here);
             * callers pass zeroed blocks, as `matmul` does. */
            continue;
        }
        const float iscale = -g_q8k_scale / max;
        for (int j = 0; j < 256; j++) {
            const float v = roundf(iscale * xs[j]);
            y[i].qs[j] = rs_as_i8(rs_min(v, 127.0f));
        }
        for (int g = 0; g < 16; g++) {
            int32_t s = 0;
            for (int t = 0; t < 16; t++) s += y[i].qs[16 * g + t];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}
/* to_float: Q/k_quants.rs:2929-2940 */
static void q8_k_to_float(const qref_q8_k *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++)
        for (int j = 0; j < 256; j++) y[256 * i + j] = x[i].d * (float)x[i].qs[j];
}

/* ---------------------------------------------------------------------- */
/* Q4_K: Q/k_quants.rs:2003-2266; helpers Q/utils.rs:50-60, 227-285        */
/* ---------------------------------------------------------------------- */
/* get_scale_min_k4: Q/utils.rs:50-60 */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* make_qkx1_quants(nmax, ntry, x[n]): Q/utils.rs:227-285 -> (scale, -min). */
static void make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *out_scale,
                             float *out_negmin) {
    uint8_t l[256];
    memset(l, 0, (size_t)n);
    /* min_by / max_by under total_cmp */
    float min = x[0], max = x[0];
    int32_t kmin = total_key(x[0]), kmax = kmin;
    for (int i = 1; i < n; i++) {
        const int32_t k = total_key(x[i]);
        if (k < kmin) { kmin = k; min = x[i]; }
        if (k >= kmax) { kmax = k; max = x[i]; }
    }
    if (max == min) {
        *out_scale = 0.0f;
        *out_negmin = 0.0f;
        return;
    }
    min = rs_min(min, 0.0f);
    float iscale = (float)nmax / (max - min);
    float scale = 1.0f / iscale;
    for (int itry = 0; itry < ntry; itry++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; i++) {
            const int32_t li = clamp_i32(nearest_int(iscale * (x[i] - min)), 0, nmax);
            if ((uint8_t)li != l[i]) { l[i] = (uint8_t)li; did_change = 1; }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *out_scale = scale;
    *out_negmin = -min;
}

/* from_float: Q/k_quants.rs:2113-2171 */
static void q4_k_from_float(const float *xall, qref_q4_k *blocks, int64_t nb) {
    for (int64_t ib = 0; ib < nb; ib++) {
        const float *x = xall + 256 * ib;
        qref_q4_k *b = &blocks[ib];
        float mins[8], scales[8];
        for (int j = 0; j < 8; j++) make_qkx1_quants(15, 5, x + 32 * j, 32, &scales[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) max_scale = rs_max(scales[j], max_scale);
        for (int j = 0; j < 8; j++) max_min = rs_max(mins[j], max_min);
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        memset(b->scales, 0, 12);
        for (int j = 0; j < 8; j++) {
            int32_t lsi = nearest_int(inv_scale * scales[j]);
            int32_t lmi = nearest_int(inv_min * mins[j]);
            const uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
            const uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
            if (j < 4) {
                b->scales[j] = ls;
                b->scales[j + 4] = lm;
            } else {
                b->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                b->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                b->scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        b->d = qref_f32_to_f16(max_scale / 63.0f);
        b->dmin = qref_f32_to_f16(max_min / 63.0f);
        uint8_t L[256];
        memset(L, 0, sizeof L);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j, b->scales, &sc, &m);
            const float d = qref_f16_to_f32(b->d) * (float)sc;
            if (d != 0.0f) {
                const float dm = qref_f16_to_f32(b->dmin) * (float)m;
                for (int ii = 0; ii < 32; ii++) {
                    const int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                    L[32 * j + ii] = (uint8_t)clamp_i32(lv, 0, 15);
                }
            }
        }
        for (int j = 0; j < 256; j += 64)
            for (int l = 0; l < 32; l++)
                b->qs[(j / 64) * 32 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}
/* to_float: Q/k_quants.rs:2238-2265 */
static void q4_k_to_float(const qref_q4_k *xs, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const qref_q4_k *b = &xs[i];
        const float d = qref_f16_to_f32(b->d), min = qref_f16_to_f32(b->dmin);
        float *out = y + 256 * i;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            const uint8_t *q = b->qs + j / 2;
            uint8_t sc, m;
            get_scale_min_k4(is, b->scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = min * (float)m;
            get_scale_min_k4(is + 1, b->scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) *out++ = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) *out++ = d2 * (float)(q[l] >> 4) - m2;
            is += 2;
        }
    }
}
/* vec_dot_unopt: Q/k_quants.rs:2031-2111 */
static float q4_k_dot_unopt(int64_t nb, const qref_q4_k *xs, const qref_q8_k *ys) {
    const uint32_t kmask1 = 0x3f3f3f3f, kmask2 = 0x0f0f0f0f, kmask3 = 0x03030303;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const qref_q4_k *x = &xs[i];
        const qref_q8_k *y = &ys[i];
        int8_t aux8[256];
        int32_t aux32[8] = {0};
        for (int j = 0; j < 4; j++) {
            for (int l = 0; l < 32; l++) aux8[64 * j + l] = (int8_t)(x->qs[32 * j + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * j + 32 + l] = (int8_t)(x->qs[32 * j + l] >> 4);
        }
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12);
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        const uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        uint8_t scales[8], mins[8];
        memcpy(scales, &utmp[0], 8);
        memcpy(mins, &utmp[2], 8);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        const int8_t *a = aux8;
        const int8_t *q8 = y->qs;
        for (int s = 0; s < 8; s++) {
            const int32_t scale = scales[s];
            for (int t = 0; t < 4; t++) {
                int16_t aux16[8];
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)((int16_t)q8[l] * (int16_t)a[l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * (int32_t)aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = qref_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        const float dmin = qref_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float tail = -0.0f;
    for (int l = 0; l < 8; l++) tail += sums[l];
    return sumf + tail;
}

/* ---------------------------------------------------------------------- */
/* Q6_K: Q/k_quants.rs:2570-2842; make_qx_quants Q/utils.rs:62-225          */
/* ---------------------------------------------------------------------- */
/* make_qx_quants(n, nmax, x, ls, rmse_type, qw=NULL): Q/utils.rs:62-225 */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *ls, int rmse_type) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) ls[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) {
            const int32_t l = nearest_int(iscale * x[i]);
            ls[i] = (int8_t)(nmax + clamp_i32(l, -nmax, nmax - 1));
        }
        return 1.0f / iscale;
    }
    const int weight_type = rmse_type % 2;
#define QX_W(xv) (weight_type == 1 ? (xv) * (xv) : 1.0f)
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        const float xv = x[i];
        int32_t l = nearest_int(iscale * xv);
        l = clamp_i32(l, -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        const float w = QX_W(xv);
        const float lf = (float)l;
        sumlx += w * xv * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        const float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            const float xv = x[i];
            int32_t l = nearest_int(is2 * xv);
            l = clamp_i32(l, -nmax, nmax - 1);
            if (l + nmax != (int32_t)ls[i]) changed = 1;
            const float w = QX_W(xv);
            const float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            const int32_t l = nearest_int(is2 * x[i]);
            ls[i] = (int8_t)(nmax + clamp_i32(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
    }
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            const float xv = x[i];
            const float w = QX_W(xv);
            const int32_t l = (int32_t)ls[i] - nmax;
            float slx = sumlx - w * xv * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int32_t new_l = nearest_int(xv * sl2 / slx);
                new_l = clamp_i32(new_l, -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * xv * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = (int8_t)(nmax + new_l);
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    if (rmse_type < 3) return scale;
    for (int is = -4; is < 4; is++) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        float slx = 0.0f, sl2 = 0.0f;
        for (int i = 0; i < n; i++) {
            const float xv = x[i];
            int32_t l = nearest_int(iscale * xv);
            l = clamp_i32(l, -nmax, nmax - 1);
            const float w = QX_W(xv);
            const float lf = (float)l;
            slx += w * xv * lf;
            sl2 += w * lf * lf;
        }
        if (sl2 > 0.0f && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) {
                const int32_t l = nearest_int(iscale * x[i]);
                ls[i] = (int8_t)(nmax + clamp_i32(l, -nmax, nmax - 1));
            }
            scale = slx / sl2;
            best = scale * slx;
        }
    }
#undef QX_W
    return scale;
}

/* from_float: Q/k_quants.rs:2657-2727 */
static void q6_k_from_float(const float *xall, qref_q6_k *ys, int64_t nb) {
    int8_t L[256];
    memset(L, 0, sizeof L);
    float scales[16];
    for (int64_t ib = 0; ib < nb; ib++) {
        const float *x = xall + 256 * ib;
        qref_q6_k *y = &ys[ib];
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int g = 0; g < 16; g++) {
            const float scale = make_qx_quants(16, 32, x + 16 * g, L + 16 * g, 1);
            scales[g] = scale;
            const float as = fabsf(scale);
            if (as > max_abs_scale) { max_abs_scale = as; max_scale = scale; }
        }
        const float iscale = -128.0f / max_scale;
        y->d = qref_f32_to_f16(1.0f / iscale);
        for (int g = 0; g < 16; g++) {
            const int32_t v = nearest_int(iscale * scales[g]);
            y->scales[g] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            const float d = qref_f16_to_f32(y->d) * (float)y->scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                const int32_t ll = clamp_i32(nearest_int(x[16 * j + ii] / d), -32, 31);
                L[16 * j + ii] = (int8_t)(ll + 32);
            }
        }
        uint8_t *ql = y->ql, *qh = y->qh;
        for (int j = 0; j < 256; j += 128) {
            for (int l = 0; l < 32; l++) {
                const uint8_t q1 = (uint8_t)(L[j + l] & 0xF);
                const uint8_t q2 = (uint8_t)(L[j + l + 32] & 0xF);
                const uint8_t q3 = (uint8_t)(L[j + l + 64] & 0xF);
                const uint8_t q4 = (uint8_t)(L[j + l + 96] & 0xF);
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                  ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}
/* to_float: Q/k_quants.rs:2810-2841 */
static void q6_k_to_float(const qref_q6_k *xs, float *yall, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const qref_q6_k *x = &xs[i];
        const float d = qref_f16_to_f32(x->d);
        for (int n = 0; n < 256; n += 128) {
            const int idx = n / 128;
            float *y = yall + 256 * i + n;
            const int8_t *sc = x->scales + 8 * idx;
            const uint8_t *ql = x->ql + 64 * idx;
            const uint8_t *qh = x->qh + 32 * idx;
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                const int8_t q2 = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                const int8_t q3 = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                const int8_t q4 = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                y[l] = d * (float)sc[is] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}
/* vec_dot_unopt: Q/k_quants.rs:2598-2655 */
static float q6_k_dot_unopt(int64_t nb, const qref_q6_k *xs, const qref_q8_k *ys) {
    float sums[8] = {0};
    for (int64_t i = 0; i < nb; i++) {
        const qref_q6_k *x = &xs[i];
        const qref_q8_k *y = &ys[i];
        int8_t aux8[256];
        float aux32[8] = {0};
        for (int j = 0; j < 256; j += 128) {
            const uint8_t *q4 = x->ql + j / 2;
            const uint8_t *qh = x->qh + j / 4;
            for (int l = 0; l < 32; l++) {
                aux8[j + l] = (int8_t)(((q4[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                aux8[j + l + 32] = (int8_t)(((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                aux8[j + l + 64] = (int8_t)(((q4[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                aux8[j + l + 96] = (int8_t)(((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
        }
        for (int j = 0; j < 16; j++) {
            const float scale = (float)x->scales[j];
            const int8_t *q8 = y->qs + 16 * j;
            const int8_t *a8 = aux8 + 16 * j;
            int16_t aux16[8];
            for (int l = 0; l < 8; l++) aux16[l] = (int16_t)((int16_t)q8[l] * (int16_t)a8[l]);
            for (int l = 0; l < 8; l++) aux32[l] += scale * (float)aux16[l];
            for (int l = 0; l < 8; l++) aux16[l] = (int16_t)((int16_t)q8[8 + l] * (int16_t)a8[8 + l]);
            for (int l = 0; l < 8; l++) aux32[l] += scale * (float)aux16[l];
        }
        const float d = qref_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* ---------------------------------------------------------------------- */
/* MXFP4: Q/k_quants.rs:429-528                                            */
/* ---------------------------------------------------------------------- */
/* mxfp4_block_dot: Q/k_quants.rs:434-442 */
float qref_mxfp4_block_dot(const qref_mxfp4 *x, const qref_q8_0 *y) {
    const float d = qref_f16_to_f32(y->d) * e8m0_to_f32_half(x->e);
    int32_t s1 = 0, s2 = 0;
    for (int j = 0; j < 16; j++) {
        s1 += (int32_t)y->qs[j] * MXFP4_VALUES[x->qs[j] & 0x0F];
        s2 += (int32_t)y->qs[j + 16] * MXFP4_VALUES[x->qs[j] >> 4];
    }
    return d * (float)(s1 + s2);
}
/* best_index_mxfp4: Q/k_quants.rs:446-457 */
static uint8_t mxfp4_best_index(float x, float d) {
    uint8_t best = 0;
    float best_err = fabsf((float)MXFP4_VALUES[0] * d - x);
    for (int i = 1; i < 16; i++) {
        const float err = fabsf((float)MXFP4_VALUES[i] * d - x);
        if (err < best_err) { best = (uint8_t)i; best_err = err; }
    }
    return best;
}
/* from_float: Q/k_quants.rs:483-506 (log2f: the libm call f32::log2 makes). */
static void mxfp4_from_float(const float *x, qref_mxfp4 *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float *xs = x + 32 * i;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(xs[j])) amax = fabsf(xs[j]);
        const uint8_t e = amax > 0.0f ? rs_as_u8(floorf(log2f(amax)) - 2.0f + 127.0f) : 0;
        const float d = e8m0_to_f32_half(e);
        y[i].e = e;
        for (int j = 0; j < 16; j++)
            y[i].qs[j] = (uint8_t)(mxfp4_best_index(xs[j], d) | (mxfp4_best_index(xs[16 + j], d) << 4));
    }
}
/* to_float: Q/k_quants.rs:465-479 */
static void mxfp4_to_float(const qref_mxfp4 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = e8m0_to_f32_half(x[i].e);
        for (int j = 0; j < 16; j++) {
            y[32 * i + j] = (float)MXFP4_VALUES[x[i].qs[j] & 0x0F] * d;
            y[32 * i + j + 16] = (float)MXFP4_VALUES[x[i].qs[j] >> 4] * d;
        }
    }
}
/* vec_dot_unopt: Q/k_quants.rs:517-527 */
static float mxfp4_dot_unopt(int64_t nb, const qref_mxfp4 *x, const qref_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) sumf += qref_mxfp4_block_dot(&x[i], &y[i]);
    return sumf;
}

/* ---------------------------------------------------------------------- */
/* IQ4_NL: Q/k_quants.rs:530-765                                           */
/* ---------------------------------------------------------------------- */
/* iq4_nl_block_dot: Q/k_quants.rs:535-543 */
float qref_iq4_nl_block_dot(const qref_iq4_nl *x, const qref_q8_0 *y) {
    const float d = qref_f16_to_f32(y->d) * qref_f16_to_f32(x->d);
    int32_t s1 = 0, s2 = 0;
    for (int j = 0; j < 16; j++) {
        s1 += (int32_t)y->qs[j] * IQ4NL_VALUES[x->qs[j] & 0x0F];
        s2 += (int32_t)y->qs[j + 16] * IQ4NL_VALUES[x->qs[j] >> 4];
    }
    return d * (float)(s1 + s2);
}
/* best_index_int8: Q/k_quants.rs:565-587 */
static uint8_t iq4_best_index(float x) {
    if (x <= (float)IQ4NL_VALUES[0]) return 0;
    if (x >= (float)IQ4NL_VALUES[15]) return 15;
    int ml = 0, mu = 15;
    while (mu - ml > 1) {
        const int mav = (ml + mu) / 2;
        if (x < (float)IQ4NL_VALUES[mav]) mu = mav; else ml = mav;
    }
    return (uint8_t)((x - (float)IQ4NL_VALUES[mu - 1] < (float)IQ4NL_VALUES[mu] - x) ? mu - 1 : mu);
}
/* quantize_iq4_impl for one IQ4_NL block (super_block 32, ntry -1):
 * Q/k_quants.rs:605-701. `l` carries the levels between blocks. */
static void iq4_nl_quantize_block(const float *xb, qref_iq4_nl *out, uint8_t *l) {
    const float GROUP_MAX_EPS = 1e-15f;
    float weight[32];
    memset(out->qs, 0, 16);
    out->d = qref_f32_to_f16(0.0f);
    float scale0;
    for (int j = 0; j < 32; j++) weight[j] = xb[j] * xb[j];
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; j++) {
        if (fabsf(xb[j]) > amax) { amax = fabsf(xb[j]); max = xb[j]; }
    }
    if (amax < GROUP_MAX_EPS) {
        scale0 = 0.0f;
    } else {
        const float v0 = (float)IQ4NL_VALUES[0];
        float d = max / v0; /* ntry <= 0 */
        const float id = 1.0f / d;
        float sumqx = 0.0f, sumq2 = 0.0f;
        for (int j = 0; j < 32; j++) {
            const uint8_t level = iq4_best_index(id * xb[j]);
            l[j] = level;
            const float q = (float)IQ4NL_VALUES[level];
            const float w = weight[j];
            sumqx += w * q * xb[j];
            sumq2 += w * q * q;
        }
        d = sumq2 > 0.0f ? sumqx / sumq2 : 0.0f;
        /* the nudged-scale loop runs over -ntry..=ntry = 1..=-1: empty */
        scale0 = d;
    }
    out->d = qref_f32_to_f16(scale0);
    for (int j = 0; j < 16; j++) out->qs[j] = (uint8_t)(l[j] | (l[16 + j] << 4));
}
/* from_float: Q/k_quants.rs:727-743 */
static void iq4_nl_from_float(const float *x, qref_iq4_nl *y, int64_t nb) {
    uint8_t l[32];
    memset(l, 0, sizeof l);
    for (int64_t i = 0; i < nb; i++) iq4_nl_quantize_block(x + 32 * i, &y[i], l);
}
/* to_float: Q/k_quants.rs:709-723 */
static void iq4_nl_to_float(const qref_iq4_nl *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = qref_f16_to_f32(x[i].d);
        for (int j = 0; j < 16; j++) {
            y[32 * i + j] = d * (float)IQ4NL_VALUES[x[i].qs[j] & 0x0F];
            y[32 * i + j + 16] = d * (float)IQ4NL_VALUES[x[i].qs[j] >> 4];
        }
    }
}
/* vec_dot_unopt: Q/k_quants.rs:754-764 */
static float iq4_nl_dot_unopt(int64_t nb, const qref_iq4_nl *x, const qref_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) sumf += qref_iq4_nl_block_dot(&x[i], &y[i]);
    return sumf;
}

/* ---------------------------------------------------------------------- */
/* generic entry points                                                     */
/* ---------------------------------------------------------------------- */
int qref_from_float(int type, const float *x, void *blocks, int64_t n) {
    const int qk = qref_block_size(type);
    if (qk == 0 || n < 0 || n % qk) return -1;
    const int64_t nb = n / qk;
    switch (type) {
    case QREF_Q4_0: q4_0_from_float(x, blocks, nb); return 0;
    case QREF_Q8_0: q8_0_from_float(x, blocks, nb); return 0;
    case QREF_Q4_K: q4_k_from_float(x, blocks, nb); return 0;
    case QREF_Q6_K: q6_k_from_float(x, blocks, nb); return 0;
    case QREF_Q8_K: q8_k_from_float(x, blocks, nb); return 0;
    case QREF_MXFP4: mxfp4_from_float(x, blocks, nb); return 0;
    case QREF_IQ4_NL: iq4_nl_from_float(x, blocks, nb); return 0;
    default: return -1;
    }
}

int qref_to_float(int type, const void *blocks, float *y, int64_t n) {
    const int qk = qref_block_size(type);
    if (qk == 0 || n < 0 || n % qk) return -1;
    const int64_t nb = n / qk;
    switch (type) {
    case QREF_Q4_0: q4_0_to_float(blocks, y, nb); return 0;
    case QREF_Q8_0: q8_0_to_float(blocks, y, nb); return 0;
    case QREF_Q4_K: q4_k_to_float(blocks, y, nb); return 0;
    case QREF_Q6_K: q6_k_to_float(blocks, y, nb); return 0;
    case QREF_Q8_K: q8_k_to_float(blocks, y, nb); return 0;
    case QREF_MXFP4: mxfp4_to_float(blocks, y, nb); return 0;
    case QREF_IQ4_NL: iq4_nl_to_float(blocks, y, nb); return 0;
    default: return -1;
    }
}

float qref_vec_dot_unopt(int type, int64_t n, const void *xs, const void *ys) {
    const int qk = qref_block_size(type);
    if (qk == 0) return NAN;
    const int64_t nb = n / qk;
    switch (type) {
    case QREF_Q4_0: return q4_0_dot_unopt(nb, xs, ys);
    case QREF_Q8_0: return q8_0_dot_unopt(nb, xs, ys);
    case QREF_Q4_K: return q4_k_dot_unopt(nb, xs, ys);
    case QREF_Q6_K: return q6_k_dot_unopt(nb, xs, ys);
    case QREF_MXFP4: return mxfp4_dot_unopt(nb, xs, ys);
    case QREF_IQ4_NL: return iq4_nl_dot_unopt(nb, xs, ys);
    default: return NAN;
    }
}
