/*
 * qref_matmul.c — candle's CPU matmul driver, `k_quants::matmul`
 * (vendor/candle/candle-core/src/quantized/k_quants.rs:2944-3065), with
 * OpenMP standing in for rayon. Work partition follows the reference (m = 1:
 * columns in chunks of 128-512; m > 1: ROW_BLOCK = 128 rows x COL_BLOCK = 64
 * columns through the several-row kernels, then a transpose). Every output
 * is one vec_dot / vec_dot_rows over the same operands, so the bits do not
 * depend on the thread count.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + CPU baseline), see qref.h.
 */
#include "qref.h"

#include <omp.h>
#include <stdlib.h>
#include <string.h>

enum { ROW_BLOCK = 128, COL_BLOCK = 64 };

static int pick_threads(int threads) { return threads > 0 ? threads : omp_get_num_procs(); }

int qref_quantize_rows(int type, int64_t m, int64_t k, const float *x, void *xq, int threads) {
    const int vt = qref_vec_dot_type(type);
    const int qk = qref_block_size(vt);
    if (vt == 0 || k % qk) return -1;
    const int64_t kb = k / qk;
    const size_t row_bytes = (size_t)kb * (size_t)qref_type_size(vt);
    memset(xq, 0, (size_t)m * row_bytes); /* `vec![zeros(); m * kb]` */
    if (m == 1) return qref_from_float(vt, x, xq, k);
    int rc = 0;
#pragma omp parallel for num_threads(pick_threads(threads)) schedule(static) reduction(| : rc)
    for (int64_t r = 0; r < m; r++) rc |= qref_from_float(vt, x + r * k, (char *)xq + r * row_bytes, k);
    return rc;
}

int qref_matmul_prequantized(int type, int64_t m, int64_t k, int64_t n, const void *xq, const void *w,
                             float *dst, int threads) {
    const int qk = qref_block_size(type);
    const int vt = qref_vec_dot_type(type);
    if (qk == 0 || k % qk || m <= 0 || n <= 0) return -1;
    const int64_t kb = k / qk;
    const size_t wrow = (size_t)kb * (size_t)qref_type_size(type);
    const size_t xrow = (size_t)kb * (size_t)qref_type_size(vt);
    const char *wb = (const char *)w;
    const char *xb = (const char *)xq;
    const int nt = pick_threads(threads);
    if (m == 1) {
        /* with_min_len(128).with_max_len(512): chunks of 128-512 columns */
#pragma omp parallel for num_threads(nt) schedule(dynamic, 256)
        for (int64_t c = 0; c < n; c++) dst[c] = qref_vec_dot(type, k, wb + c * wrow, xb);
        return 0;
    }
    float *dst_t = (float *)malloc((size_t)n * (size_t)m * sizeof(float));
    if (!dst_t) return -1;
    for (int64_t row_base = 0; row_base < m; row_base += ROW_BLOCK) {
        const int rows = (int)(m - row_base < ROW_BLOCK ? m - row_base : ROW_BLOCK);
        const char *lhs_blk = xb + (size_t)row_base * xrow;
        const int64_t nblk = (n + COL_BLOCK - 1) / COL_BLOCK;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
        for (int64_t blk = 0; blk < nblk; blk++) {
            const int64_t c_end = (blk + 1) * COL_BLOCK < n ? (blk + 1) * COL_BLOCK : n;
            for (int64_t c = blk * COL_BLOCK; c < c_end; c++)
                qref_vec_dot_rows(type, k, wb + c * wrow, lhs_blk, rows, dst_t + c * m + row_base, 0);
        }
    }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < m; r++)
        for (int64_t c = 0; c < n; c++) dst[r * n + c] = dst_t[c * m + r];
    free(dst_t);
    return 0;
}

int qref_matmul(int type, int64_t m, int64_t k, int64_t n, const float *x, const void *w, float *dst,
                int threads) {
    const int vt = qref_vec_dot_type(type);
    const int qk = qref_block_size(type);
    if (vt == 0 || qk == 0 || k % qk || m <= 0) return -1;
    const size_t bytes = (size_t)m * (size_t)(k / qk) * (size_t)qref_type_size(vt);
    void *xq = malloc(bytes);
    if (!xq) return -1;
    int rc = qref_quantize_rows(type, m, k, x, xq, threads);
    if (rc == 0) rc = qref_matmul_prequantized(type, m, k, n, xq, w, dst, threads);
    free(xq);
    return rc;
}

/* examples/qmatmul_bench.rs:19-40: batch row outer, one vec_dot per element. */
int qref_matmul_upstream(int type, int64_t m, int64_t k, int64_t n, const float *x, const void *w,
                         float *dst) {
    const int vt = qref_vec_dot_type(type);
    const int qk = qref_block_size(type);
    if (vt == 0 || qk == 0 || k % qk || m <= 0) return -1;
    const int64_t kb = k / qk;
    const size_t xrow = (size_t)kb * (size_t)qref_type_size(vt);
    const size_t wrow = (size_t)kb * (size_t)qref_type_size(type);
    char *xq = (char *)calloc((size_t)m, xrow);
    if (!xq) return -1;
    for (int64_t r = 0; r < m; r++) qref_from_float(vt, x + r * k, xq + r * xrow, k);
    for (int64_t r = 0; r < m; r++)
        for (int64_t c = 0; c < n; c++)
            dst[r * n + c] = qref_vec_dot(type, k, (const char *)w + c * wrow, xq + r * xrow);
    free(xq);
    return 0;
}
