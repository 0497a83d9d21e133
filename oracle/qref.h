/*
 * qref — CPU restatement of candle's quantized-matmul path, as SwarmLLM
 * vendors it. TEST INFRASTRUCTURE ONLY: the parity oracle for the HIP
 * library and the timed CPU baseline. No product code may link or call it.
 *
 * Reference (paths relative to the reference checkout,
 * Q/ = vendor/candle/candle-core/src/quantized/):
 *   block layouts        Q/k_quants.rs:201-317
 *   from_float/to_float  Q/k_quants.rs (per type, cited at each function)
 *   scalar vec_dot_unopt Q/k_quants.rs (per type)
 *   AVX2 vec_dot(+rows)  Q/avx.rs (per type)
 *   matmul driver        Q/k_quants.rs:2944-3065
 *   quantizer helpers    Q/utils.rs:1-285
 *
 * Arithmetic follows the reference operation for operation: no FP
 * contraction (the build passes -ffp-contract=off; Rust never fuses), FMA
 * only where the reference calls an FMA intrinsic, f16 conversions IEEE
 * round-to-nearest-even (the `half` 2.7.1 crate).
 *
 * Parity status per function is recorded in the test files under tests/
 * (test_oracle_*.py); each function below names what pins it.
 */
#ifndef QREF_H
#define QREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (Q/mod.rs:319-371). */
enum {
    QREF_Q4_0 = 2,
    QREF_Q8_0 = 8,
    QREF_Q4_K = 12,
    QREF_Q6_K = 14,
    QREF_Q8_K = 15,
    QREF_IQ4_NL = 20,
    QREF_MXFP4 = 39,
};

/* Block layouts: Q/k_quants.rs:165-317 (repr(C), natural alignment). */
typedef struct { uint16_t d; uint8_t qs[16]; } qref_q4_0;                 /* 18 B / 32  */
typedef struct { uint16_t d; int8_t qs[32]; } qref_q8_0;                  /* 34 B / 32  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } qref_q4_k; /* 144 B / 256 */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } qref_q6_k; /* 210 B / 256 */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } qref_q8_k;  /* 292 B / 256 */
typedef struct { uint8_t e; uint8_t qs[16]; } qref_mxfp4;                 /* 17 B / 32  */
typedef struct { uint16_t d; uint8_t qs[16]; } qref_iq4_nl;               /* 18 B / 32  */

/* ---- registry ---------------------------------------------------------- */
int qref_block_size(int type);       /* values per block, 0 if unknown */
int qref_type_size(int type);        /* bytes per block, 0 if unknown  */
int qref_vec_dot_type(int type);     /* the activation block type a weight type dots against */

/* ---- f16 (half 2.7.1: IEEE binary16, RNE) ------------------------------ */
uint16_t qref_f32_to_f16(float x);
float qref_f16_to_f32(uint16_t h);

/* ---- quantize / dequantize (n = element count, a multiple of the block) - */
/* Generic entry points; `type` is a GGUF id above. Return 0, or -1 for an
 * unknown type or a count that is not a whole number of blocks. */
int qref_from_float(int type, const float *x, void *blocks, int64_t n);
int qref_to_float(int type, const void *blocks, float *y, int64_t n);

/* SWARMLLM_Q8K_SCALE (Q/k_quants.rs:145-152): the magnitude a Q8_K block's
 * largest activation is written at, 127 (default) or 128 (candle before #404). */
void qref_set_q8k_scale(float s);

/* ---- dot products: weight blocks `xs` against activation blocks `ys` ---- */
/* vec_dot_unopt (scalar generic) and vec_dot (the AVX2 kernel a
 * target-cpu=native x86 build runs). n = element count. */
float qref_vec_dot_unopt(int type, int64_t n, const void *xs, const void *ys);
float qref_vec_dot(int type, int64_t n, const void *xs, const void *ys);
/* vec_dot_rows_chosen: one weight column against `rows` activation rows
 * stored contiguously; per_row != 0 forces the per-row loop
 * (SWARMLLM_QMATMUL_ROWS=per-row). Bit-identical either way. */
void qref_vec_dot_rows(int type, int64_t n, const void *xs, const void *ys, int rows,
                       float *out, int per_row);

/* ---- matmul driver: k_quants::matmul (Q/k_quants.rs:2944-3065) --------- */
/* dst[m][n] = x[m][k] · Wᵀ, W = n rows of k values in blocks of `type`.
 * threads <= 0 uses every core; the bits never depend on it. */
int qref_matmul(int type, int64_t m, int64_t k, int64_t n, const float *x,
                const void *w, float *dst, int threads);
/* The same product with the activation already quantized (VecDotType
 * blocks, m rows of k/block values): the driver after its quantize step. */
int qref_matmul_prequantized(int type, int64_t m, int64_t k, int64_t n, const void *xq,
                             const void *w, float *dst, int threads);
/* The upstream ordering (row outer, one vec_dot per element), the exactness
 * reference of examples/qmatmul_bench.rs:19-40. */
int qref_matmul_upstream(int type, int64_t m, int64_t k, int64_t n, const float *x,
                         const void *w, float *dst);
/* The activation quantization step of the driver (VecDotType from_float per row). */
int qref_quantize_rows(int type, int64_t m, int64_t k, const float *x, void *xq, int threads);

/* Q8_0 hidden-state wire codec (src/inference/quant.rs:1-107), qref_wire.c:
 * bytes of n values (ceil(n/32)*34, -1 if it overflows), encode, decode
 * (-1 when nbytes is not qref_wire_bytes(n)). */
int64_t qref_wire_bytes(int64_t n);
void qref_wire_encode(const float *values, int64_t n, uint8_t *out);
int qref_wire_decode(const uint8_t *bytes, int64_t nbytes, int64_t n, float *out);

/* gated activations act(gate) * up (qref_glu.c) */
void qref_silu_mul(const float *gate, const float *up, float *out, int64_t n);
void qref_swiglu_oai_mul(const float *gate, const float *up, float *out, int64_t n);
void qref_gelu_mul(const float *gate, const float *up, float *out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
