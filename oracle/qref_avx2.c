/*
 * qref_avx2.c — the AVX2 dot products a target-cpu=native x86 build of the
 * reference runs (Q/avx.rs, Q/ = vendor/candle/candle-core/src/quantized/),
 * restated intrinsic for intrinsic so the f32 results carry the same bits:
 * single-row kernels and the several-row kernels (bit-identical to the
 * single-row ones by construction: every row keeps its own accumulators and
 * sees the single-row sequence of operations).
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + CPU baseline), see qref.h.
 * Built with -mavx2 -mfma -mf16c -ffp-contract=off.
 */
#include "qref.h"

#include <immintrin.h>
#include <string.h>

float qref_mxfp4_block_dot(const qref_mxfp4 *x, const qref_q8_0 *y);
float qref_iq4_nl_block_dot(const qref_iq4_nl *x, const qref_q8_0 *y);

static const int8_t IQ4NL_VALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1, 13, 25, 38, 53, 69, 89, 113};
static const int8_t MXFP4_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* ---- helpers: Q/avx.rs:14-52, 334-339 ---------------------------------- */
static inline __m256 sum_i16_pairs_float(__m256i x) {
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), x));
}
static inline __m256 mul_sum_us8_pairs_float(__m256i ax, __m256i sy) {
    return sum_i16_pairs_float(_mm256_maddubs_epi16(ax, sy));
}
static inline float hsum_float_8(__m256 x) {
    __m128 res = _mm256_extractf128_ps(x, 1);
    res = _mm_add_ps(res, _mm256_castps256_ps128(x));
    res = _mm_add_ps(res, _mm_movehl_ps(res, res));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}
static inline __m256i bytes_from_nibbles_32(const uint8_t *p) {
    const __m128i tmp = _mm_loadu_si128((const __m128i *)p);
    const __m256i bytes = _mm256_insertf128_si256(_mm256_castsi128_si256(tmp), _mm_srli_epi16(tmp, 4), 1);
    return _mm256_and_si256(_mm256_set1_epi8(0xF), bytes);
}
static inline __m256 mul_sum_i8_pairs_float(__m256i x, __m256i y) {
    const __m256i ax = _mm256_sign_epi8(x, x);
    const __m256i sy = _mm256_sign_epi8(y, x);
    return mul_sum_us8_pairs_float(ax, sy);
}
/* scale_product / block_scale_products lane: f16(x) * f16(y) in f32, broadcast. */
static inline __m256 scale_product(uint16_t x, uint16_t y) {
    const __m128 both = _mm_cvtph_ps(_mm_cvtsi32_si128((int)((uint32_t)x | ((uint32_t)y << 16))));
    return _mm256_broadcastss_ps(_mm_mul_ss(both, _mm_movehdup_ps(both)));
}
static inline float f16(uint16_t h) { return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h))); }
static inline __m256i set_m128i(__m128i hi, __m128i lo) {
    return _mm256_insertf128_si256(_mm256_castsi128_si256(lo), hi, 1);
}
/* get_scale_shuffle (Q/avx.rs:521-530): 16-byte chunk i = (2i) x8, (2i+1) x8. */
static inline __m128i get_scale_shuffle(int i) {
    return _mm_set_epi8(2 * i + 1, 2 * i + 1, 2 * i + 1, 2 * i + 1, 2 * i + 1, 2 * i + 1, 2 * i + 1, 2 * i + 1,
                        2 * i, 2 * i, 2 * i, 2 * i, 2 * i, 2 * i, 2 * i, 2 * i);
}
/* get_scale_shuffle_k4 (Q/avx.rs:533-548): 32-byte chunk i = (2i, 2i+1) x16. */
static inline __m256i get_scale_shuffle_k4(int i) {
    return _mm256_set1_epi16((short)((2 * i) | ((2 * i + 1) << 8)));
}

/* ---- 32-value formats: column-side unpack (Q/avx.rs:373-404) ------------ */
static inline __m256i q8_0_bytes(const qref_q8_0 *x) { return _mm256_loadu_si256((const __m256i *)x->qs); }
static inline __m256i q4_0_bytes(const qref_q4_0 *x) {
    return _mm256_sub_epi8(bytes_from_nibbles_32(x->qs), _mm256_set1_epi8(8));
}

/* vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0: Q/avx.rs:53-87 */
static float dot_q8_0(int64_t nb, const qref_q8_0 *xs, const qref_q8_0 *ys) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < nb; i++) {
        const __m256 d = scale_product(xs[i].d, ys[i].d);
        const __m256 q = mul_sum_i8_pairs_float(q8_0_bytes(&xs[i]), _mm256_loadu_si256((const __m256i *)ys[i].qs));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_float_8(acc);
}
static float dot_q4_0(int64_t nb, const qref_q4_0 *xs, const qref_q8_0 *ys) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < nb; i++) {
        const __m256 d = scale_product(xs[i].d, ys[i].d);
        const __m256 q = mul_sum_i8_pairs_float(q4_0_bytes(&xs[i]), _mm256_loadu_si256((const __m256i *)ys[i].qs));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_float_8(acc);
}

/* Several-row pass of a signed 32-value format: Q/avx.rs:417-440 (the
 * `signed` arm of rows_of_a_32_value_format!). R <= 4 rows. */
#define ROWS_32_SIGNED(NAME, BLK, UNPACK)                                                        \
    static void NAME(int64_t nb, const BLK *xs, const qref_q8_0 *ys, int R, float *out) {        \
        __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),          \
                         _mm256_setzero_ps()};                                                   \
        for (int64_t bi = 0; bi < nb; bi++) {                                                    \
            const __m256i bx = UNPACK(&xs[bi]);                                                  \
            const __m256i ax = _mm256_sign_epi8(bx, bx);                                         \
            for (int r = 0; r < R; r++) {                                                        \
                const qref_q8_0 *y = &ys[r * nb + bi];                                           \
                const __m256 d = scale_product(xs[bi].d, y->d);                                  \
                const __m256i by = _mm256_loadu_si256((const __m256i *)y->qs);                   \
                const __m256 q = mul_sum_us8_pairs_float(ax, _mm256_sign_epi8(by, bx));          \
                acc[r] = _mm256_fmadd_ps(d, q, acc[r]);                                          \
            }                                                                                    \
        }                                                                                        \
        for (int r = 0; r < R; r++) out[r] = hsum_float_8(acc[r]);                               \
    }
ROWS_32_SIGNED(pass_q8_0, qref_q8_0, q8_0_bytes)
ROWS_32_SIGNED(pass_q4_0, qref_q4_0, q4_0_bytes)

/* ---- MXFP4 / IQ4_NL: Q/avx.rs:95-169 ------------------------------------ */
static inline __m256i lut_bytes(const int8_t *table, const uint8_t *qs) {
    const __m128i values = _mm_loadu_si128((const __m128i *)table);
    const __m128i m4b = _mm_set1_epi8(0x0F);
    const __m128i q4bits = _mm_loadu_si128((const __m128i *)qs);
    const __m128i low = _mm_shuffle_epi8(values, _mm_and_si128(q4bits, m4b));
    const __m128i high = _mm_shuffle_epi8(values, _mm_and_si128(_mm_srli_epi16(q4bits, 4), m4b));
    return set_m128i(high, low);
}
static inline float e8m0_half(uint8_t e) {
    const uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
/* mxfp4_scale (Q/avx.rs:264-269): f16(y) * half(e). */
static inline __m256 mxfp4_scale(uint8_t e, uint16_t y) { return _mm256_set1_ps(f16(y) * e8m0_half(e)); }

static float dot_mxfp4(int64_t nb, const qref_mxfp4 *xs, const qref_q8_0 *ys) {
    __m256 accum1 = _mm256_setzero_ps(), accum2 = _mm256_setzero_ps();
    int64_t ib = 0;
    for (; ib + 1 < nb; ib += 2) {
        const __m256i by0 = _mm256_loadu_si256((const __m256i *)ys[ib].qs);
        const __m256i by1 = _mm256_loadu_si256((const __m256i *)ys[ib + 1].qs);
        const __m256 p0 = mul_sum_i8_pairs_float(lut_bytes(MXFP4_VALUES, xs[ib].qs), by0);
        const __m256 p1 = mul_sum_i8_pairs_float(lut_bytes(MXFP4_VALUES, xs[ib + 1].qs), by1);
        accum1 = _mm256_fmadd_ps(mxfp4_scale(xs[ib].e, ys[ib].d), p0, accum1);
        accum2 = _mm256_fmadd_ps(mxfp4_scale(xs[ib + 1].e, ys[ib + 1].d), p1, accum2);
    }
    float sumf = hsum_float_8(_mm256_add_ps(accum1, accum2));
    if (ib < nb) sumf += qref_mxfp4_block_dot(&xs[ib], &ys[ib]);
    return sumf;
}
static float dot_iq4_nl(int64_t nb, const qref_iq4_nl *xs, const qref_q8_0 *ys) {
    __m256 accum1 = _mm256_setzero_ps(), accum2 = _mm256_setzero_ps();
    int64_t ib = 0;
    for (; ib + 1 < nb; ib += 2) {
        const __m256i by0 = _mm256_loadu_si256((const __m256i *)ys[ib].qs);
        const __m256i by1 = _mm256_loadu_si256((const __m256i *)ys[ib + 1].qs);
        const __m256 p0 = mul_sum_i8_pairs_float(lut_bytes(IQ4NL_VALUES, xs[ib].qs), by0);
        const __m256 p1 = mul_sum_i8_pairs_float(lut_bytes(IQ4NL_VALUES, xs[ib + 1].qs), by1);
        accum1 = _mm256_fmadd_ps(scale_product(xs[ib].d, ys[ib].d), p0, accum1);
        accum2 = _mm256_fmadd_ps(scale_product(xs[ib + 1].d, ys[ib + 1].d), p1, accum2);
    }
    float sumf = hsum_float_8(_mm256_add_ps(accum1, accum2));
    if (ib < nb) sumf += qref_iq4_nl_block_dot(&xs[ib], &ys[ib]);
    return sumf;
}

/* ---- Q6_K: Q/avx.rs:550-643 (single) and 668-813 (rows) ----------------- */
/* The single-row kernel is the R = 1 pass: each row's sequence is the same. */
static void pass_q6_k(int64_t nb, const qref_q6_k *xs, const qref_q8_k *ys, int R, float *out) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m256i m2 = _mm256_set1_epi8(3);
    const __m256i m32s = _mm256_set1_epi8(32);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (int64_t bi = 0; bi < nb; bi++) {
        const qref_q6_k *x = &xs[bi];
        const float xd = f16(x->d);
        const __m128i scales = _mm_loadu_si128((const __m128i *)x->scales);
        const uint8_t *q4 = x->ql;
        const uint8_t *qh = x->qh;
        const int8_t *q8p[4];
        float ds[4];
        for (int r = 0; r < R; r++) {
            const qref_q8_k *y = &ys[r * nb + bi];
            q8p[r] = y->qs;
            ds[r] = y->d * xd;
        }
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(),
                           _mm256_setzero_si256()};
        for (int j = 0; j < 2; j++) {
            const int is = j * 4;
            const __m256i sc_0 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, get_scale_shuffle(is)));
            const __m256i sc_1 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, get_scale_shuffle(is + 1)));
            const __m256i sc_2 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, get_scale_shuffle(is + 2)));
            const __m256i sc_3 = _mm256_cvtepi8_epi16(_mm_shuffle_epi8(scales, get_scale_shuffle(is + 3)));
            const __m256i q4bits1 = _mm256_loadu_si256((const __m256i *)q4);
            q4 += 32;
            const __m256i q4bits2 = _mm256_loadu_si256((const __m256i *)q4);
            q4 += 32;
            const __m256i q4bits_h = _mm256_loadu_si256((const __m256i *)qh);
            qh += 32;
            const __m256i q4h_0 = _mm256_slli_epi16(_mm256_and_si256(q4bits_h, m2), 4);
            const __m256i q4h_1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 2), m2), 4);
            const __m256i q4h_2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 4), m2), 4);
            const __m256i q4h_3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(q4bits_h, 6), m2), 4);
            const __m256i q4_0 = _mm256_or_si256(_mm256_and_si256(q4bits1, m4), q4h_0);
            const __m256i q4_1 = _mm256_or_si256(_mm256_and_si256(q4bits2, m4), q4h_1);
            const __m256i q4_2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits1, 4), m4), q4h_2);
            const __m256i q4_3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits2, 4), m4), q4h_3);
            for (int r = 0; r < R; r++) {
                const int8_t *q8 = q8p[r];
                const __m256i q8_0 = _mm256_loadu_si256((const __m256i *)q8);
                const __m256i q8_1 = _mm256_loadu_si256((const __m256i *)(q8 + 32));
                const __m256i q8_2 = _mm256_loadu_si256((const __m256i *)(q8 + 64));
                const __m256i q8_3 = _mm256_loadu_si256((const __m256i *)(q8 + 96));
                q8p[r] = q8 + 128;
                const __m256i q8s_0 = _mm256_maddubs_epi16(m32s, q8_0);
                const __m256i q8s_1 = _mm256_maddubs_epi16(m32s, q8_1);
                const __m256i q8s_2 = _mm256_maddubs_epi16(m32s, q8_2);
                const __m256i q8s_3 = _mm256_maddubs_epi16(m32s, q8_3);
                __m256i p16_0 = _mm256_maddubs_epi16(q4_0, q8_0);
                __m256i p16_1 = _mm256_maddubs_epi16(q4_1, q8_1);
                __m256i p16_2 = _mm256_maddubs_epi16(q4_2, q8_2);
                __m256i p16_3 = _mm256_maddubs_epi16(q4_3, q8_3);
                p16_0 = _mm256_sub_epi16(p16_0, q8s_0);
                p16_1 = _mm256_sub_epi16(p16_1, q8s_1);
                p16_2 = _mm256_sub_epi16(p16_2, q8s_2);
                p16_3 = _mm256_sub_epi16(p16_3, q8s_3);
                p16_0 = _mm256_madd_epi16(sc_0, p16_0);
                p16_1 = _mm256_madd_epi16(sc_1, p16_1);
                p16_2 = _mm256_madd_epi16(sc_2, p16_2);
                p16_3 = _mm256_madd_epi16(sc_3, p16_3);
                sumi[r] = _mm256_add_epi32(sumi[r], _mm256_add_epi32(p16_0, p16_1));
                sumi[r] = _mm256_add_epi32(sumi[r], _mm256_add_epi32(p16_2, p16_3));
            }
        }
        for (int r = 0; r < R; r++)
            acc[r] = _mm256_fmadd_ps(_mm256_set1_ps(ds[r]), _mm256_cvtepi32_ps(sumi[r]), acc[r]);
    }
    for (int r = 0; r < R; r++) out[r] = hsum_float_8(acc[r]);
}

/* ---- Q4_K: Q/avx.rs:1297-1381 (single) and 1383-1528 (rows) ------------- */
static void pass_q4_k(int64_t nb, const qref_q4_k *xs, const qref_q8_k *ys, int R, float *out) {
    const uint32_t kmask1 = 0x3f3f3f3f, kmask2 = 0x0f0f0f0f, kmask3 = 0x03030303;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    __m128 acc_m[4] = {_mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps()};
    for (int64_t bi = 0; bi < nb; bi++) {
        const qref_q4_k *x = &xs[bi];
        const float xd = f16(x->d), xdmin = f16(x->dmin);
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12);
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        const uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        const __m256i mins_and_scales =
            _mm256_cvtepu8_epi16(_mm_set_epi32((int)utmp[3], (int)utmp[2], (int)utmp[1], (int)utmp[0]));
        const __m128i mins = _mm256_extracti128_si256(mins_and_scales, 1);
        const __m128i sc128 = _mm256_extracti128_si256(mins_and_scales, 0);
        const __m256i scales = set_m128i(sc128, sc128);
        float ds[4];
        const int8_t *q8p[4];
        for (int r = 0; r < R; r++) {
            const qref_q8_k *y = &ys[r * nb + bi];
            ds[r] = y->d * xd;
            const float dmin = -y->d * xdmin;
            const __m256i q8sums = _mm256_loadu_si256((const __m256i *)y->bsums);
            const __m128i q8s =
                _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
            const __m128i prod = _mm_madd_epi16(mins, q8s);
            acc_m[r] = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m[r]);
            q8p[r] = y->qs;
        }
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(),
                           _mm256_setzero_si256()};
        const uint8_t *q4 = x->qs;
        for (int j = 0; j < 4; j++) {
            const __m256i scale_l = _mm256_shuffle_epi8(scales, get_scale_shuffle_k4(2 * j));
            const __m256i scale_h = _mm256_shuffle_epi8(scales, get_scale_shuffle_k4(2 * j + 1));
            const __m256i q4bits = _mm256_loadu_si256((const __m256i *)q4);
            q4 += 32;
            const __m256i q4l = _mm256_and_si256(q4bits, m4);
            const __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            for (int r = 0; r < R; r++) {
                const __m256i q8l = _mm256_loadu_si256((const __m256i *)q8p[r]);
                __m256i p16l = _mm256_maddubs_epi16(q4l, q8l);
                p16l = _mm256_madd_epi16(scale_l, p16l);
                sumi[r] = _mm256_add_epi32(sumi[r], p16l);
                const __m256i q8h = _mm256_loadu_si256((const __m256i *)(q8p[r] + 32));
                __m256i p16h = _mm256_maddubs_epi16(q4h, q8h);
                p16h = _mm256_madd_epi16(scale_h, p16h);
                sumi[r] = _mm256_add_epi32(sumi[r], p16h);
                q8p[r] += 64;
            }
        }
        for (int r = 0; r < R; r++)
            acc[r] = _mm256_fmadd_ps(_mm256_set1_ps(ds[r]), _mm256_cvtepi32_ps(sumi[r]), acc[r]);
    }
    for (int r = 0; r < R; r++) {
        __m128 am = _mm_add_ps(acc_m[r], _mm_movehl_ps(acc_m[r], acc_m[r]));
        am = _mm_add_ss(am, _mm_movehdup_ps(am));
        out[r] = hsum_float_8(acc[r]) + _mm_cvtss_f32(am);
    }
}

/* ---- dispatch ----------------------------------------------------------- */
float qref_vec_dot(int type, int64_t n, const void *xs, const void *ys) {
    const int qk = qref_block_size(type);
    if (qk == 0) return __builtin_nanf("");
    const int64_t nb = n / qk;
    float out;
    switch (type) {
    case QREF_Q4_0: return dot_q4_0(nb, xs, ys);
    case QREF_Q8_0: return dot_q8_0(nb, xs, ys);
    case QREF_Q4_K: pass_q4_k(nb, xs, ys, 1, &out); return out;
    case QREF_Q6_K: pass_q6_k(nb, xs, ys, 1, &out); return out;
    case QREF_MXFP4: return dot_mxfp4(nb, xs, ys);
    case QREF_IQ4_NL: return dot_iq4_nl(nb, xs, ys);
    default: return __builtin_nanf("");
    }
}

/* Types with a several-row kernel; MXFP4 and IQ4_NL take the generic
 * per-row loop (no vec_dot_rows override in Q/k_quants.rs:459-765). */
static int has_pass(int type) {
    return type == QREF_Q4_0 || type == QREF_Q8_0 || type == QREF_Q4_K || type == QREF_Q6_K;
}
static void run_pass(int type, int64_t nb, const void *xs, const void *ys, int R, float *out) {
    switch (type) {
    case QREF_Q4_0: pass_q4_0(nb, xs, ys, R, out); break;
    case QREF_Q8_0: pass_q8_0(nb, xs, ys, R, out); break;
    case QREF_Q4_K: pass_q4_k(nb, xs, ys, R, out); break;
    case QREF_Q6_K: pass_q6_k(nb, xs, ys, R, out); break;
    default: break;
    }
}

/* vec_dot_rows_chosen (Q/k_quants.rs:124-140) over the per-type
 * vec_dot_rows (Q/avx.rs:466-508, 668-700, 1397-1436). */
void qref_vec_dot_rows(int type, int64_t n, const void *xs, const void *ys, int rows, float *out,
                       int per_row) {
    const int qk = qref_block_size(type);
    const int vsz = qref_type_size(qref_vec_dot_type(type));
    const int64_t nb = n / qk;
    const char *yb = (const char *)ys;
    if (per_row || !has_pass(type)) {
        for (int r = 0; r < rows; r++) out[r] = qref_vec_dot(type, n, xs, yb + (size_t)r * nb * vsz);
        return;
    }
    int r0 = 0;
    while (r0 + 4 <= rows) {
        run_pass(type, nb, xs, yb + (size_t)r0 * nb * vsz, 4, out + r0);
        r0 += 4;
    }
    const int left = rows - r0; /* tail_in_one_pass, Q/avx.rs:660-666 */
    if (left == 2 || left == 3) {
        run_pass(type, nb, xs, yb + (size_t)r0 * nb * vsz, left, out + r0);
        return;
    }
    for (int r = r0; r < rows; r++) out[r] = qref_vec_dot(type, n, xs, yb + (size_t)r * nb * vsz);
}
