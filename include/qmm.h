/*
 * qmm.h — C ABI of libqmm: quantized matrix products over GGUF block
 * formats (Q8_0, Q4_K, Q6_K, IQ4_NL, MXFP4) on AMD Instinct MI355X (gfx950).
 *
 * It is the drop-in device arm below candle's QTensor / QMatMul::forward as
 * SwarmLLM vendors it. The entry points and their conventions follow the C
 * ABI the reference already binds from Rust for its card kernels
 * (vendor/candle/candle-kernels/src/ffi.rs:58-107, implemented in
 * vendor/candle/candle-kernels/src/ggml_mmq/mmq_entry.cu:100-223) and the
 * device-arm surface QCudaStorage exposes
 * (vendor/candle/candle-core/src/quantized/dummy_cuda.rs:10-143):
 *   - every call returns an int status (QMM_OK ... ) and never aborts;
 *   - buffers are raw device pointers the caller allocates and owns;
 *     the library allocates nothing and frees nothing;
 *   - `stream` is a hipStream_t passed as int64 (0 = the null stream);
 *   - weight types are GGUF type ids; weights are the bytes a GGUF holds
 *     (row-major [n][k], k a multiple of the block size);
 *   - outputs are fully overwritten (callers need not zero them);
 *   - stale runtime errors are cleared before a launch, so a failure
 *     reported is this call's own.
 *
 * Outputs: dst[r][j] = sum_i x[r][i] * W[j][i] for activation rows r and
 * weight rows j, row-major [rows][n] with leading dimension `ldd` (>= n).
 */
#ifndef QMM_H
#define QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the swarm_mmq_status values
 * (vendor/candle/candle-kernels/src/ggml_mmq/swarm_mmq.cuh:85-93), plus NO_ROOM. */
enum qmm_status {
    QMM_OK = 0,
    QMM_UNSUPPORTED = 1,          /* type or shape not covered                    */
    QMM_WORKSPACE_TOO_SMALL = 2,  /* the caller's workspace is under *need        */
    QMM_DEVICE_ERROR = 3,         /* a HIP runtime call or launch failed          */
    QMM_NO_TILE = 4,              /* no kernel configuration fits this device     */
    QMM_NO_ROOM = 5,              /* fault injection: this product must fall back */
};

/* GGUF type ids this library covers (vendor/candle/candle-core/src/quantized/mod.rs:319-371). */
enum qmm_type {
    QMM_Q8_0 = 8,
    QMM_Q4_K = 12,
    QMM_Q6_K = 14,
    QMM_IQ4_NL = 20,
    QMM_MXFP4 = 39,
};

/* Activation layouts (qmm_act_layout).
 *   QMM_ACT_Q8K:  per 256 values, the codes / f32 scale / 16-value sums of
 *                 candle's BlockQ8K::from_float (k_quants.rs:2882-2927);
 *   QMM_ACT_Q8_0: per 32 values, the codes / f16 scale of
 *                 BlockQ8_0::from_float (k_quants.rs:1240-1269), with each
 *                 block's exact code sum.
 * Both hold those values bit for bit, stored as planes (codes, scales,
 * sums; see qmm_act_planes) rather than interleaved structs. */
enum qmm_act_layout_id { QMM_ACT_Q8K = 0, QMM_ACT_Q8_0 = 1 };

/* 1 when the library's kernels run on the current device (gfx950), else 0.
 * Replaces swarm_mmq_available (mmq_entry.cu:100-117). */
int qmm_available(void);

/* The activation layout a product of `rows` activation rows against a weight
 * of `type` reads, or -1 for a type not covered. Products whose layouts agree
 * can share one quantized activation (QMatMul::forward_shared).
 * Replaces swarm_mmq_q8_1_layout (mmq_entry.cu:130-135). */
int qmm_act_layout(int type, int64_t rows);

/* Bytes of a quantized activation of `rows` x `k` in `layout`.
 * Replaces swarm_mmq_q8_1_bytes (mmq_entry.cu:137-141). */
size_t qmm_act_bytes(int layout, int64_t k, int64_t rows);

/* Byte offsets of the planes inside an activation buffer: codes (int8
 * [rows][k]), scales (f32 [rows][k/256] or [rows][k/32]) and sums (int16
 * [rows][k/16] for QMM_ACT_Q8K, int32 [rows][k/32] for QMM_ACT_Q8_0). */
int qmm_act_planes(int layout, int64_t k, int64_t rows, size_t *codes_off, size_t *scales_off,
                   size_t *sums_off);

/* Quantize `rows` f32 rows of `k` values (`stride` floats apart) into `xq`
 * in `layout`. Replaces swarm_mmq_quantize (mmq_entry.cu:144-158); the
 * codes and scales are bit-exact to candle's CPU from_float. */
int qmm_quantize_act(const float *x, void *xq, int layout, int64_t k, int64_t rows, int64_t stride,
                     int64_t stream);

/* Largest `rows` qmm_matvec takes in one launch. */
int qmm_matvec_max_rows(void);

/* dst = x · Wᵀ for 1 <= rows <= qmm_matvec_max_rows(), from an activation
 * already quantized in qmm_act_layout(type, rows): the fused dequant + dot
 * decode kernel. Replaces the reference's vector kernels
 * mul_mat_vec_*_q8_1_cuda (launched from quantized/cuda.rs:519-620). */
int qmm_matvec(int type, const void *w, const void *xq, float *dst, int64_t ldd, int64_t k, int64_t n,
               int64_t rows, int64_t stream);

/* dst = x · Wᵀ for any rows >= 1 from an activation already quantized in
 * qmm_act_layout(type, rows) (qmm_quantize_act), the kernel picked by the
 * reference's few-rows policy (quantized/cuda.rs:775-839): the decode
 * kernels up to qmm_matvec_max_rows() rows; for Q4_K and Q6_K the few-row
 * int8 matrix-core kernels from 4 rows on weights of 2 MiB or more and for
 * 9-32 rows, then the int8 matrix-core GEMMs from 33 rows; for Q8_0, IQ4_NL
 * and MXFP4 the int8 matrix-core GEMM from 9 rows. Nothing is allocated.
 * The SWARMLLM_QMATMUL_MMQ switches below move these lines. Replaces
 * swarm_mmq_matmul's launch step (mmq_entry.cu:162-203), which multiplies
 * the activation swarm_mmq_quantize produced. */
int qmm_matmul(int type, const void *w, const void *xq, float *dst, int64_t ldd, int64_t k, int64_t n,
               int64_t rows, int64_t stream);

/* The reference's A/B switches for the matrix-core line, read from the
 * environment once per process (quantized/cuda.rs:737-872):
 *   SWARMLLM_QMATMUL_MMQ=dp4a|0|off|false: no matrix-core kernel; products
 *     run on the decode kernels, qmm_matvec_max_rows() rows a launch;
 *   SWARMLLM_QMATMUL_MMQ_MAX_ROWS=N: the matrix-core kernels take at most N rows;
 *   SWARMLLM_QMATMUL_MMQ_MIN_ROWS=N: one few-rows line for every type;
 *   SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES=B: the least weight bytes of a
 *     few-rows product (0: any);
 *   SWARMLLM_QMATMUL_MMQ_CAPTURED=0|off|false: products of at most
 *     qmm_matvec_max_rows() rows on a stream being captured stay on the
 *     decode kernels.
 * qmm_mmq_few_rows_line gives a type's line as this process reads it
 * (mmq_few_rows_line, cuda.rs:850-872): products of fewest..8 rows against
 * a weight of least_bytes or more go to the matrix cores.
 * qmm_mmq_max_rows: the most rows a matrix-core kernel takes (0 when the
 * switch is off). qmm_mmq_captured: 0 when captured few-rows products stay
 * on the decode kernels. */
int qmm_mmq_few_rows_line(int type, int64_t *fewest_rows, int64_t *least_bytes);
int64_t qmm_mmq_max_rows(void);
int qmm_mmq_captured(void);

/* SWARMLLM_QMATMUL_EXACT=1|on|true (read once; no counterpart in the
 * reference): the exact Q4_K / Q6_K kernels only. Without it three kernels
 * feed the matrix cores a rounded product of a code and its sub-block scale
 * (normalised error up to about 1e-3, inside the 2e-3 bound): the
 * single-pass Q4_K and Q6_K GEMMs (from 129 rows) and the few-row Q6_K
 * kernel's single-product form (k >= 2048, from the few-rows line to 32 rows), so a product's bits
 * can depend on the row count of its batch (1-2 rows are always exact). With
 * it every row count sums exact int32 products, at the exact kernels' speed.
 * qmm_exact_forms: 1 when the switch is on. */
int qmm_exact_forms(void);

/* set_force_dmmv (quantized/cuda.rs:29-33): while on, qmm_forward,
 * qmm_forward_shared and qmm_forward_glu dequantize each weight value (as
 * qmm_dequantize does) against the f32 activation and sum in f32, without
 * quantizing the activation: the reference's dequantize_mul_mat_vec and
 * dequantize + f32 matmul path (cuda.rs:1653-1745). Grouped products and the
 * entry points that take a quantized activation are not affected. */
void qmm_set_force_dmmv(int on);
int qmm_force_dmmv(void);

/* Set-up a product's first launch would otherwise do, done ahead of a HIP
 * graph capture: the current device's properties, the LDS limit of every
 * kernel of the library that asks for more than 64 KiB, and the
 * no-allocation scratch's address (qmm_forward_noalloc). Launches nothing.
 * On a stream being captured, a product of at most qmm_matvec_max_rows()
 * rows takes a matrix-core kernel only once its type is prepared on the
 * current device (else the decode kernels serve it); the first such product
 * outside a capture prepares its type itself. Returns QMM_UNSUPPORTED for a
 * type not covered, QMM_NO_TILE off gfx950. qmm_prepared: 1 once `type` is
 * prepared on the current device. Replaces swarm_mmq_prepare_few_rows
 * (mmq_entry.cu:204-223) as mmq_prepare_few_rows_once calls it
 * (quantized/cuda.rs:890-932). */
int qmm_prepare(int type);
int qmm_prepared(int type);

/* QMatMul::accumulate_in_f32 / QCudaStorage::accumulate_in_f32
 * (quantized/mod.rs:1187-1200, quantized/cuda.rs:1375-1380): keep a weight's
 * products in f32 where a card's prompt pass would accumulate them in f16.
 * Every product of this library sums in int32 and f32 already, so this
 * changes nothing: QMM_OK for a covered type, QMM_UNSUPPORTED otherwise. */
int qmm_accumulate_in_f32(int type);

/* dst = x · Wᵀ for any rows, from an f32 activation: quantizes it into the
 * workspace and picks the kernel by rows (the QCudaStorage::fwd policy,
 * quantized/cuda.rs:1653-1680). With launch == 0 nothing is enqueued and
 * *need is set to the workspace bytes the launch will want; with
 * launch != 0 the product is enqueued, and QMM_WORKSPACE_TOO_SMALL is
 * returned (nothing enqueued) when workspace_bytes is less than the
 * quantized activation. For a single-pass Q4_K GEMM whose tiles fill at
 * most half the CUs, *need also counts the slots of a K split (the product
 * cut into 2 or 4 parts along K, added in part order); with a workspace that
 * holds the activation but not those slots the product runs uncut.
 * Replaces the plan/launch pair of swarm_mmq_matmul (mmq_entry.cu:162-203). */
int qmm_forward(int type, const void *w, const float *x, int64_t x_stride, float *dst, int64_t ldd,
                void *workspace, size_t workspace_bytes, size_t *need, int64_t k, int64_t n, int64_t rows,
                int launch, int64_t stream);

/* qmm_forward without a workspace: the activation scratch is a 16 MiB
 * device array the library holds per GPU until the process ends
 * (qmm_forward_noalloc_max_bytes()). No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); the entry
 * point itself allocates nothing. Products whose quantized activation
 * exceeds the scratch return QMM_WORKSPACE_TOO_SMALL with nothing enqueued.
 * Results equal, bit for bit, qmm_forward's with a workspace of
 * qmm_forward_noalloc_max_bytes() bytes: so qmm_forward's with the
 * workspace it plans (*need) whenever that need fits the scratch. A larger
 * planned need (a single-pass GEMM's K-split slots beside the activation,
 * e.g. 4096 x 4096 at 512 rows) runs as qmm_forward does with a workspace
 * that holds the activation only: Q4_K uncut, Q6_K on its exact GEMM. All
 * calls on one GPU share the scratch: calls that overlap on one GPU (other
 * streams, other threads) race on it. */
int qmm_forward_noalloc(int type, const void *w, const float *x, int64_t x_stride, float *dst, int64_t ldd,
                        int64_t k, int64_t n, int64_t rows, int64_t stream);
size_t qmm_forward_noalloc_max_bytes(void);

/* dst[i] = x · W[i]ᵀ for `count` weights of one type and the same k that
 * share the activation x (rows x k f32, `x_stride` floats apart): the
 * activation is quantized once for all of them. Weight i has n[i] rows and
 * writes dst[i] with leading dimension ldd[i]. For Q4_K and Q6_K at 1-2
 * rows the products run as one launch per 4 weights, each quantizing the
 * activation in LDS (workspace unused); otherwise the activation is
 * quantized once into the workspace and each weight's product reads it, the
 * weights the few-row matrix-core kernels or the single-pass Q4_K GEMM take
 * sharing one launch per 4 (each weight's K split as its own forward would
 * choose, so results equal qmm_forward's bit for bit). Plan (launch == 0) and
 * launch as qmm_forward. Replaces QMatMul::forward_shared with the CUDA
 * arm's shared activation (quantized/mod.rs:1221-1263,
 * quantized/cuda.rs:622-720). */
int qmm_forward_shared(int type, int count, const void *const *w, const int64_t *n, float *const *dst,
                       const int64_t *ldd, const float *x, int64_t x_stride, void *workspace,
                       size_t workspace_bytes, size_t *need, int64_t k, int64_t rows, int launch,
                       int64_t stream);

/* Gated activations of an MLP: act(gate) * up. */
enum qmm_glu_act_id {
  QMM_GLU_SILU = 0,       /* gate / (1 + exp(-gate)) * up (fast_math.rs:48-60) */
  QMM_GLU_SWIGLU_OAI = 1, /* min(gate, 7) sharpened by 1.702, times clamp(up, -7, 7) + 1 (fast_math.rs:84-104) */
  QMM_GLU_GELU = 2        /* tanh-form GELU of gate, times up (fast_math.rs:62-76) */
};

/* dst[r][j] = act(x_r · gate_j) * (x_r · up_j): an MLP's gate and up
 * products (two weights of one type, n x k each) sharing one quantized
 * activation, and the gated activation between them, written once. For Q4_K
 * at 1-2 rows and k <= 8192 with a 16-byte aligned activation this is ONE
 * launch (each wave computes gate row j and up row j and writes the product;
 * the activation quantized in LDS); otherwise the two products run as
 * qmm_forward_shared into the workspace, followed by the elementwise GLU.
 * Either way the results equal qmm_forward_shared followed by qmm_glu bit for
 * bit. Plan (launch == 0) and launch as qmm_forward. Replaces the
 * reference's forward_shared of ffn_up and ffn_gate followed by silu_mul /
 * swiglu_oai_mul / the GELU product (src/inference/layers/mod.rs:583-632). */
int qmm_forward_glu(int type, int act, const void *w_gate, const void *w_up, const float *x, int64_t x_stride,
                    float *dst, int64_t ldd, void *workspace, size_t workspace_bytes, size_t *need, int64_t k,
                    int64_t n, int64_t rows, int launch, int64_t stream);

/* out[i] = act(gate[i]) * up[i] for n values (f32, on the device). Replaces
 * the reference's fused elementwise ops silu_mul / swiglu_oai_mul
 * (src/inference/fast_math.rs:48-130, their card kernels in
 * kernels/fused_decode.cu). */
int qmm_glu(int act, const float *gate, const float *up, float *out, int64_t n, int64_t stream);

/* Grouped expert products (mixture-of-experts layers). Routing entry i
 * (i < size_m) pairs sorted_ids[i] (a token's k-th choice, numbered
 * token * topk + k) with expert expert_ids[i]; it writes
 *   dst[p][j] = scale_p * (x[in_p] . W_e[j])   for j < n,
 * p = sorted_ids[i], e = expert_ids[i], in_p = p when topk_w is given (one
 * input row per pair, size_m rows) else p / topk (one per token, size_m/topk
 * rows), scale_p = topk_w[p] or 1. `w` holds num_experts weights of n x k
 * back to back, each in GGUF blocks of `type`: Q8_0, IQ4_NL or MXFP4 (the
 * activation quantized per 32 values, Q8_0), or Q4_K or Q6_K with k at most
 * 16384 (per 256 values, Q8_K). Entries whose expert or pair
 * is out of range write nothing. Entries with one expert read its weights
 * once when they are consecutive (ids sorted by expert); any order gives
 * the same result. Each dst[p] equals qmm_forward of x[in_p] against W_e,
 * times scale_p, bit for bit. Plan (launch == 0) and launch as qmm_forward:
 * the workspace holds the quantized activation and the routing runs.
 * Replaces moe_gemm_gguf (candle-kernels/src/moe/moe_gguf.cu:149-252,
 * which allocates its own scratch) as called from
 * src/layers/moe_card.rs:48-170, and QMatMul::matmul_many over the touched
 * experts (quantized/mod.rs:697-780). */
int qmm_moe_forward(int type, const void *w, int num_experts, const float *x, int64_t x_stride,
                    const int32_t *sorted_ids, const int32_t *expert_ids, const float *topk_w, int topk,
                    float *dst, int64_t ldd, void *workspace, size_t workspace_bytes, size_t *need, int64_t k,
                    int64_t n, int64_t size_m, int launch, int64_t stream);

/* Input types of qmm_moe_forward_prefill: the reference's input_dtype (0 f16,
 * 1 bf16), and f32, which the product rounds to f16 as the reference's caller
 * does before its launch (src/inference/layers/moe_card.rs:113-121). */
enum qmm_x_dtype { QMM_X_F16 = 0, QMM_X_BF16 = 1, QMM_X_F32 = 2 };

/* Grouped expert products of a prompt on the f16 / bf16 matrix cores. The
 * routing, `w`, scale_p, in_p and the output rows are qmm_moe_forward's; x
 * holds the input rows (x_stride values apart) as f16, bf16 or f32
 * (x_dtype). It writes
 *   dst[p][j] = scale_p * sum_i r(x[in_p][i]) * r(W_e[j][i])
 * with r the rounding to f16 (f16 or f32 input) or bf16 (bf16 input), to
 * nearest even, of each input value and of each weight value dequantized in
 * f32 as qmm_dequantize does; the products are summed in f32 in an order of
 * the kernel's (the reference's tensor-core sum: not the bits of
 * qmm_moe_forward, whose activation is quantized). Types: Q8_0, IQ4_NL, MXFP4
 * (k a multiple of 32) and Q4_K (k a multiple of 256, w 16-byte aligned),
 * Q6_K (k a multiple of 256). Entries whose expert or pair is out of range
 * write nothing; entries in any order give the same result, consecutive
 * entries of one expert (up to 64 a workgroup) read its weights together. Plan (launch == 0) and launch as qmm_forward: the
 * workspace holds the routing's run and chunk tables and a 16-bit copy of the
 * input rows (used for f32 input, or 16-bit input whose rows are not 16-byte
 * aligned). Two launches. Replaces moe_gemm_gguf_prefill
 * (candle-kernels/src/moe/moe_wmma_gguf.cu:450-535, kernel :191-371, which
 * allocates its own tables and reads expert_ids to size them), as
 * src/inference/layers/moe_card.rs:48-170 calls it for a prompt of more than
 * 8 tokens (src/inference/layers/mod.rs:2753). */
int qmm_moe_forward_prefill(int type, const void *w, int num_experts, const void *x, int x_dtype, int64_t x_stride,
                            const int32_t *sorted_ids, const int32_t *expert_ids, const float *topk_w, int topk,
                            float *dst, int64_t ldd, void *workspace, size_t workspace_bytes, size_t *need,
                            int64_t k, int64_t n, int64_t size_m, int launch, int64_t stream);

/* ---- GGUF files into device memory --------------------------------------
 * A parsed GGUF file: candle's gguf_file::Content::read
 * (quantized/gguf_file.rs:415-487): header (magic "GGUF", versions 1-3),
 * metadata key/value pairs, tensor infos (name, ggml type, dimensions
 * outermost first, offset from the tensor data), and the tensor data's start,
 * the end of the infos rounded up to general.alignment (U8/U16/U32 or a
 * non-negative I8/I16/I32 value; 32 without it). qmm_gguf_open returns
 * QMM_UNSUPPORTED with *out = NULL for a file that is not one (bad magic or
 * version, an unknown value or ggml type, a truncated header). */
typedef struct qmm_gguf qmm_gguf;
int qmm_gguf_open(const char *path, qmm_gguf **out);
void qmm_gguf_close(qmm_gguf *g);
int qmm_gguf_version(const qmm_gguf *g);
uint64_t qmm_gguf_alignment(const qmm_gguf *g);
uint64_t qmm_gguf_data_offset(const qmm_gguf *g);

/* Tensor infos (Content::tensor_infos): index by name (-1 when absent), name,
 * and type / dimensions (dims[0..3], outermost first, 1 past n_dims) / offset
 * from the data start / bytes (0 when the element count is not a whole
 * number of blocks or its bytes pass INT64_MAX, which qmm_gguf_load then
 * refuses). */
int64_t qmm_gguf_tensor_count(const qmm_gguf *g);
int64_t qmm_gguf_find_tensor(const qmm_gguf *g, const char *name);
const char *qmm_gguf_tensor_name(const qmm_gguf *g, int64_t i);
int qmm_gguf_tensor_info(const qmm_gguf *g, int64_t i, int *type, int *n_dims, int64_t *dims, uint64_t *offset,
                         uint64_t *bytes);

/* Metadata (Content::metadata) in file order (a repeated key keeps its last
 * value): key, GGUF value type (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
 * 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64; -1 for no such pair)
 * with the element type and length of an array (the type itself and 1 for a
 * scalar), and element j of it (j = 0 for a scalar): integers and bools in
 * *iv (a u64 as its bits), f32/f64 in *fv, strings in *sv (trailing NULs
 * dropped, as the reference drops them). Arrays of arrays are parsed but not
 * read element by element. */
int64_t qmm_gguf_kv_count(const qmm_gguf *g);
int64_t qmm_gguf_find_kv(const qmm_gguf *g, const char *key);
const char *qmm_gguf_kv_key(const qmm_gguf *g, int64_t i);
int qmm_gguf_kv_type(const qmm_gguf *g, int64_t i, int *elem_type, int64_t *len);
int qmm_gguf_kv_get(const qmm_gguf *g, int64_t i, int64_t j, int64_t *iv, double *fv, const char **sv);

/* Bytes of a device buffer for `nelem` values of ggml type `type`: its
 * blocks plus MATRIX_ROW_PADDING = 512 values' worth of blocks
 * (quantized/cuda.rs:43, 1846-1870); 0 for an unknown type, a count that
 * is not a whole number of blocks, or a size past INT64_MAX. */
size_t qmm_padded_bytes(int type, int64_t nelem);

/* Tensor i's bytes from the file into device memory dst (dst_bytes >=
 * qmm_padded_bytes of the tensor), the padding zeroed: ggml_file::
 * qtensor_read + cuda::load_quantized_read (ggml_file.rs:220-256,
 * cuda.rs:2025-2075), read through two pinned staging buffers of 16 MiB the
 * library keeps (a chunk is read while the previous one copies;
 * with_pinned_load_staging, cuda.rs:1966-2018). Returns when the bytes are
 * on the device; loads on one process are serialized. A tensor whose bytes
 * would run past the end of the file is refused (QMM_UNSUPPORTED) before
 * anything is copied. The reference's switches, read once:
 *   SWARMLLM_LOAD_PINNED=0: one pageable 16 MiB staging buffer, each chunk's
 *     copy finished before the next read (cuda.rs:1979-1983); also where the
 *     runtime refuses page-locked memory;
 *   SWARMLLM_LOAD_READ=fresh: the tensor read through a fresh host buffer of
 *     its whole size, copied at once (gguf_file.rs:57-63).
 * qmm_pinned_load_chunks: chunks copied through the pinned pair since the
 * process started (pinned_load_chunks, cuda.rs:1966-1972). */
int qmm_gguf_load(const qmm_gguf *g, int64_t i, void *dst, size_t dst_bytes, int64_t stream);
uint64_t qmm_pinned_load_chunks(void);

/* A stack of expert weights with only the named entries loaded: tensor i of
 * the file is [entries, ...] (dims[0] entries of one weight each, a whole
 * number of blocks); slot slots[c] (c < count) is read from the file into
 * dst at slot * entry bytes, every other slot and the padding zeroed
 * (never to be read). dst_bytes >= qmm_padded_bytes of the whole tensor.
 * A slot out of range is refused with nothing copied. The file-side form of
 * load_quantized_entries (quantized/cuda.rs:2101-2127): a processor-held
 * mixture-of-experts layer sends a chunk's chosen experts. */
int qmm_gguf_load_entries(const qmm_gguf *g, int64_t i, int64_t count, const int64_t *slots, void *dst,
                          size_t dst_bytes, int64_t stream);

/* load_quantized_entries (quantized/cuda.rs:2101-2127): a stack of `entries`
 * slots of entry_bytes (whole blocks of `type`) in dst, holding host bytes
 * parts[c] at slot slots[c], every other slot and the padding (512 values'
 * worth of blocks) zeroed; dst_bytes >= entries * entry_bytes + padding.
 * Returns when the parts have been copied (they may be released). A slot out
 * of range is refused with nothing copied. */
int qmm_load_entries(int type, int64_t entries, size_t entry_bytes, int64_t count, const int64_t *slots,
                     const void *const *parts, void *dst, size_t dst_bytes, int64_t stream);

/* load_quantized_beside (quantized/cuda.rs:2082-2099): a weight's len host
 * bytes (whole blocks of `type`) into dst, padded as a device weight, the
 * copy issued on copy_stream beside the work on `stream`, which waits for it
 * before its next work. Returns when the copy is done (the host bytes may be
 * released); work already queued on `stream` is not waited for. */
int qmm_load_beside(int type, const void *data, size_t len, void *dst, size_t dst_bytes, int64_t copy_stream,
                    int64_t stream);

/* The chosen rows of a table of GGUF blocks (an embedding lookup):
 * out[r] = table[ids[r]], row r of n_ids, each row hidden / block_size
 * blocks of `type` copied whole (the five formats, and F32 (0), F16 (1),
 * BF16 (30)). hidden must be a whole number of blocks (else
 * QMM_UNSUPPORTED), the table must hold vocab rows (table_bytes), and out
 * n_ids rows (else QMM_WORKSPACE_TOO_SMALL); qmm_gather_row_bytes gives the
 * bytes of a row. ids are u32 on the device: 0xFFFFFFFF writes a zero row
 * (index_select's "no row"), and any other id >= vocab writes a zero row and
 * adds 1 to *bad when `bad` (a u32 on the device the caller zeroes) is not
 * NULL, for the caller to refuse, as the reference's host path refuses it
 * (a row of zero bytes dequantizes to zeros in every format). Replaces
 * QTensor::gather_rows / QCudaStorage::gather_rows (quantized/mod.rs:
 * 1039-1091, quantized/cuda.rs:1478-1540). */
int qmm_gather_row_bytes(int type, int64_t hidden, size_t *row_bytes);
int qmm_gather_rows(int type, const void *table, size_t table_bytes, int64_t vocab, int64_t hidden,
                    const uint32_t *ids, int64_t n_ids, void *out, size_t out_bytes, uint32_t *bad, int64_t stream);

/* Dequantize `nelem` values of weight type `type` into f32 (out_f16 == 0)
 * or IEEE f16 (out_f16 != 0; each value is f16 of the f32 one).
 * Replaces QCudaStorage::dequantize / dequantize_f16
 * (dummy_cuda.rs:44-52; kernels quantized.cu:828-1230). */
int qmm_dequantize(int type, const void *w, void *out, int out_f16, int64_t nelem, int64_t stream);

/* Quantize `nelem` f32 values on the device into GGUF blocks of `type`,
 * bit-exact to candle's from_float (QTensor::quantize / quantize_onto,
 * dummy_cuda.rs:54-70). `scratch` must hold qmm_quantize_scratch_bytes(). */
size_t qmm_quantize_scratch_bytes(int type, int64_t nelem);
int qmm_quantize_weights(int type, const float *x, void *w, int64_t nelem, void *scratch,
                         size_t scratch_bytes, int64_t stream);

/* Bytes of `nelem` values of `type` in GGUF blocks (GgmlDType::type_size x
 * elements / block_size, quantized/mod.rs:421-461); 0 for a type not covered
 * or a count that is not a whole number of blocks. */
size_t qmm_type_bytes(int type, int64_t nelem);
int qmm_block_size(int type);

/* The Q8_0 hidden-state wire codec: the bytes in which a layer split sends
 * activations between the peers holding consecutive layers. Per 32 values
 * [f16 scale][32 x i8], a partial trailing group zero-padded; the block
 * maximum skips non-finite values and codes are clamped to [-127, 127].
 * Bit-exact to the reference's codec.
 * qmm_wire_bytes: ceil(n / 32) * 34, or 0 when n < 0 or the size would not
 * fit (q8_0_byte_len_checked, src/inference/quant.rs:98-104).
 * qmm_wire_encode: replaces quantize_q8_0 (src/inference/quant.rs:24-60);
 * `out` holds qmm_wire_bytes(n) bytes.
 * qmm_wire_decode: replaces dequantize_q8_0 (src/inference/quant.rs:65-92);
 * QMM_UNSUPPORTED (nothing enqueued) when in_bytes != qmm_wire_bytes(n). */
size_t qmm_wire_bytes(int64_t n);
int qmm_wire_encode(const float *x, int64_t n, void *out, int64_t stream);
int qmm_wire_decode(const void *in, size_t in_bytes, int64_t n, float *out, int64_t stream);

/* The bare streaming read a product's weight bytes are measured against (a
 * measurement aid; no counterpart in the reference): one launch that reads
 * a_bytes at a and b_bytes at b once (16-byte aligned spans, sizes multiples
 * of 16), 1024 workgroups of 512 threads in 16-byte nontemporal loads, and
 * writes one word per workgroup to sink (qmm_read_floor_sink_bytes()). Its
 * duration over a weight's bytes is the floor a one-launch product of that
 * weight is held against. */
size_t qmm_read_floor_sink_bytes(void);
int qmm_read_floor(const void *a, size_t a_bytes, const void *b, size_t b_bytes, void *sink, int64_t stream);

/* Fault injection, host side (the reference's fail_the_next_mmq_allocation,
 * quantized/cuda.rs:972-991): the next qmm_forward launch returns
 * QMM_NO_ROOM without enqueuing anything, once. */
void qmm_fail_next_launch(void);

/* Synthetic data: `n` f32 values from N(mean, std) on the device,
 * reproducible from `seed` (splitmix64 counters, Box-Muller in double). */
int qmm_fill_normal(float *out, int64_t n, uint64_t seed, float mean, float std, int64_t stream);

/* Kernel launches enqueued by this library since the process started
 * (the evidence of which kernel ran, like mmq_mma_products,
 * quantized/cuda.rs:937-945): matvec launches, GEMM launches, grouped
 * expert products (qmm_moe_forward) and prompt grouped products
 * (qmm_moe_forward_prefill). */
uint64_t qmm_matvec_launches(void);
uint64_t qmm_gemm_launches(void);
uint64_t qmm_moe_launches(void);
uint64_t qmm_moe_prefill_launches(void);

/* The launcher of the last kernel this library enqueued, with its template
 * arguments (a static string, "" before any launch): which instantiation
 * served a product, as the reference's tests read mmq_mma_products
 * (quantized/cuda.rs:937-945). Process-wide; the last writer wins. */
const char *qmm_last_kernel(void);

#ifdef __cplusplus
}
#endif
#endif /* QMM_H */
