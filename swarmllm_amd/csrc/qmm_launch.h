// qmm_launch.h — host-side launchers of libqmm's kernels (internal to the
// library; the public C ABI is include/qmm.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qmm {

// The name of the last kernel launcher this library ran (its signature with
// template arguments), read by qmm_last_kernel: the evidence of which kernel
// instantiation served a product.
void note_launch(const char* what);
#define QMM_NOTE_LAUNCH() ::qmm::note_launch(__PRETTY_FUNCTION__)

// ---- activation layouts on the device --------------------------------------
// The codes, scales and sums are bit-for-bit those of candle's BlockQ8K /
// BlockQ8_0 from_float; only their placement differs: planes, 16-B aligned.
//   ACT_Q8K (per 256, for Q4_K / Q6_K, decode and the MFMA GEMM):
//     codes  int8  [rows][k]
//     d      f32   [rows][k/256]
//     bsums  int16 [rows][k/16]
//   ACT_Q8_0 (per 32, for Q8_0 / MXFP4 / IQ4_NL, products and grouped experts):
//     codes  int8  [rows][k]
//     d      f32   [rows][k/32]   (the f16 scale, widened exactly)
//     sums   int32 [rows][k/32]   (exact sum of the block's codes)
enum ActLayout : int { ACT_Q8K = 0, ACT_Q8_0 = 1 };

struct ActPlanes {
  int8_t* codes;
  float* d;
  void* sums;  // int16 (ACT_Q8K) or int32 (ACT_Q8_0)
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Byte size of an activation of `rows` x `k` in `layout`, and its planes.
size_t act_bytes(int layout, int64_t k, int64_t rows);
ActPlanes act_planes(int layout, void* base, int64_t k, int64_t rows);
// The byte offsets of the scales and sums planes (the codes start at 0).
void act_plane_offsets(int layout, int64_t k, int64_t rows, size_t* scales_off, size_t* sums_off);

// ---- launchers (return hipSuccess or the launch error) ---------------------
hipError_t launch_act_quantize(int layout, const float* x, int64_t stride, int64_t k, int64_t rows,
                               void* out, float q8k_scale, hipStream_t s);
// The activation quantization of a grouped expert product (layout ACT_Q8_0
// for the 32-value formats, ACT_Q8K for Q4_K and Q6_K), which also writes its
// run table (1 + 3 size_m ints) from expert_ids in the same launch.
hipError_t launch_act_quantize_moe(int layout, const float* x, int64_t stride, int64_t k, int64_t rows, void* out,
                                   const int32_t* expert_ids, int64_t size_m, int32_t* runs, float q8k_scale,
                                   hipStream_t s);
hipError_t launch_weight_quantize(int type, const float* x, void* w, int64_t nelem, void* scratch,
                                  hipStream_t s);
size_t weight_quantize_scratch_bytes(int type, int64_t nelem);
hipError_t launch_dequantize(int type, const void* w, void* out, int out_f16, int64_t nelem, hipStream_t s);
// dst = x · Wᵀ with each weight value dequantized (to_float) and the f32
// activation unquantized, summed in f32: the set_force_dmmv path.
hipError_t launch_dmmv(int type, const void* w, int64_t n, int64_t k, const float* x, int64_t xstride, int64_t rows,
                       float* dst, int64_t ldd, hipStream_t s);
// `p` points at the first of `rows` activation rows (planes already offset).
hipError_t launch_matvec(int type, const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows,
                         float* dst, int64_t ldd, hipStream_t s);
// The planes of rows [r0, ...) of an activation laid out for `total_rows`.
ActPlanes act_rows(int layout, const ActPlanes& p, int64_t k, int64_t r0);
int matvec_max_rows();

// ---- weights sharing one activation (QMatMul::forward_shared) -------------
// Up to kMaxTargets weights of the same type and k, whose rows one launch
// numbers one after another: target t holds rows [row_end[t-1], row_end[t]).
constexpr int kMaxTargets = 4;
struct MvTargets {
  const void* w[kMaxTargets];
  float* dst[kMaxTargets];
  int64_t ldd[kMaxTargets];
  int64_t row_end[kMaxTargets];
  int count;
};

// Q4_K decode matvec over 1-2 activation rows, streaming: `waves` waves
// each walk about n_total/waves weight rows with the next row's loads in
// flight. Quantizes the f32 activation in LDS (pre == nullptr; rows 16-byte
// aligned, see mv_q4k_rows_fusable) or reads pre-quantized Q8_K planes.
bool mv_q4k_rows_supported(int64_t k, int64_t rows);
bool mv_q4k_rows_fusable(const float* x, int64_t xstride);
// Launch shape: waves in the grid, waves per workgroup (4 or 16), and
// whether a wave prefetches its next row before computing the current one.
struct MvShape {
  int64_t waves;
  int wpg;
  bool prefetch;
};
int64_t mv_q4k_rows_waves(int64_t n_total, int per_wave);

// Q6_K decode matvec over 1-2 activation rows: each wave streams whole rows
// in spans of 16 super-blocks through its LDS buffer, the next spans' loads in
// flight; one 16-wave workgroup per CU (cus), a wave per row where rows are
// few. Quantizes the f32 activation in LDS (pre == nullptr) or reads
// pre-quantized Q8_K planes.
bool mv_q6k_rows_supported(int64_t k, int64_t rows);
hipError_t launch_mv_q6k_rows(const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, float qmax, int cus, hipStream_t s);
hipError_t launch_mv_q4k_rows(const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, float qmax, const MvShape& sh, hipStream_t s);
// Q8_0 / IQ4_NL / MXFP4 decode matvec over 1-2 activation rows (mv_b32s.hip):
// each wave streams whole rows in spans of 128 blocks, the next span in
// flight; one 16-wave workgroup per CU. Quantizes the f32 activation in LDS
// (pre == nullptr; rows 16-byte aligned) or reads pre-quantized Q8_0 planes.
bool mv_b32_rows_supported(int type, int64_t k, int64_t rows);
hipError_t launch_mv_b32_rows(int type, const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, int cus, hipStream_t st);
hipError_t launch_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float std, hipStream_t s);

// ---- prefill GEMM on the int8 matrix cores --------------------------------
// dst = x · Wᵀ for a Q4_K weight from the Q8_K activation planes of `rows`
// rows (qmm_quantize_act ACT_Q8K); used from gemm_q4k_min_rows() rows up.
// Grouped expert products (moe.hip, moe_kq.hip): the types and row lengths
// covered, the activation layout each quantizes to, bytes of the run table
// for size_m routing entries, and the grouped kernel's launch from an
// activation already quantized in that layout and its run table
// (launch_act_quantize_moe).
bool moe_supported(int type, int64_t k);
int moe_act_layout(int type);
size_t moe_runs_bytes(int64_t size_m);
bool moe_kq_supported(int type, int64_t k);
hipError_t launch_moe_kq(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                         const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                         float* dst, int64_t ldd, int cus, hipStream_t st);
hipError_t launch_moe(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                      const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                      float* dst, int64_t ldd, int cus, hipStream_t st);
// MXFP4 routings of up to 256 entries, rows of up to 128 blocks: the grouped
// product in one launch, the kernel finding the runs and quantizing the f32
// input rows itself (the same codes, scales and result bits as the two-launch
// form).
bool moe_fp4_fused_takes(int type, int64_t k, int64_t size_m);
// The same for Q4_K and Q6_K routings of up to 256 entries (moe_kq.hip: the
// input rows quantized to Q8_K in LDS with qmax as launch_act_quantize_moe).
bool moe_kq_fused_takes(int type, int64_t k, int64_t size_m);
hipError_t launch_moe_kq_fused(int type, const void* w, int num_experts, int64_t n, int64_t k, const float* x,
                               int64_t x_stride, const int32_t* expert_ids, const int32_t* ids, const float* topk_w,
                               int topk, int64_t size_m, float* dst, int64_t ldd, float qmax, int cus,
                               hipStream_t st);
hipError_t launch_moe_fp4_fused(const void* w, int num_experts, int64_t n, int64_t k, const float* x,
                                int64_t x_stride, const int32_t* expert_ids, const int32_t* ids, const float* topk_w,
                                int topk, int64_t size_m, float* dst, int64_t ldd, hipStream_t st);

// Grouped expert products of prompt-size routings on the f16 / bf16 matrix
// cores (moe_pf.hip): the types and row lengths covered, a weight row's
// bytes, bytes of the chunk table, the prologue (run and chunk tables from
// expert_ids; the input rows into 16-bit values at xo when x_kind >= 0: 0 f16
// or 1 bf16 copied, 2 f32 to f16, 3 f32 to bf16) and the grouped kernel over
// 16-bit input rows (16-byte aligned, x_stride a multiple of 8).
bool moe_pf_supported(int type, int64_t k);
bool moe_pf_weights_ok(int type, const void* w);  // Q4_K: 16-byte aligned
int64_t moe_pf_row_bytes(int type, int64_t k);
size_t moe_pf_chunks_bytes(int64_t size_m);
hipError_t launch_moe_pf_prep(const int32_t* expert_ids, int64_t size_m, int32_t* runs, int32_t* chunks,
                              const void* x, int x_kind, int64_t x_stride, int64_t k, int64_t rows, uint16_t* xo,
                              int cus, hipStream_t st);
hipError_t launch_moe_pf(int type, bool bf16, const void* w, int num_experts, int64_t n, int64_t k, const uint16_t* x,
                         int64_t x_stride, const int32_t* chunks, const int32_t* ids, const float* topk_w, int topk,
                         int64_t size_m, float* dst, int64_t ldd, hipStream_t st);

// Q4_K products of a few rows (gemm_q4k_skinny.hip): up to
// gemm_q4k_skinny_max_rows() activation rows, targets as the stream kernels.
int gemm_q4k_skinny_max_rows();
bool gemm_q4k_skinny_fits(int64_t k, int64_t rows);
hipError_t launch_gemm_q4k_skinny(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, int cus,
                                  hipStream_t st);

// Q6_K products of a few rows (gemm_q6k_skinny.hip): up to 32 activation
// rows, targets as the stream kernels.
bool gemm_q6k_skinny_fits(int64_t k, int64_t rows);
hipError_t launch_gemm_q6k_skinny(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, int cus,
                                  hipStream_t st);

// The gate+up+GLU decode launch (mv_q4k.hip): Q4_K, 1-2 rows, k <= 8192;
// act is a GluAct (glu_act.h). And the elementwise GLU (glu.hip) over rows
// of n values.
bool mv_q4k_glu_supported(int64_t k, int64_t rows);
hipError_t launch_mv_q4k_glu(int act, const void* wg, const void* wu, int64_t n, int64_t k, int64_t rows,
                             const float* x, int64_t xstride, const ActPlanes* pre, float qmax, float* dst, int64_t ldd,
                             int cus, hipStream_t st);
hipError_t launch_glu(int act, const float* gate, int64_t ldg, const float* up, int64_t ldu, float* out, int64_t ldo,
                      int64_t n, int64_t rows, hipStream_t st);

// The Q8_0 hidden-state wire codec (wire.hip): bytes of n values (-1 when
// they would not fit an int64), encode, decode.
int64_t wire_bytes(int64_t n);
hipError_t launch_wire_encode(const float* x, int64_t n, void* out, hipStream_t st);
hipError_t launch_wire_decode(const void* in, int64_t n, float* out, hipStream_t st);

// The single-pass Q4_K GEMM (gemm_q4k_sp.hip), from gemm_q4k_sp_min_rows()
// rows: weights rounded into one int8 operand, 256-row tiles.
int gemm_q4k_sp_min_rows();
bool gemm_q4k_sp_fits(int64_t n, int64_t k, int64_t rows);
hipError_t launch_gemm_q4k_sp(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                              int64_t ldd, hipStream_t s);
// K splits for one weight's product (1, 2 or 4), the workspace the splits of
// a launch over `t` need (0: none split), and the launch itself: up to
// kMaxTargets weights sharing one activation in one launch; with split_ws of
// at least gemm_q4k_sp_split_bytes bytes the products that leave CUs idle are
// cut along K (their results the same whatever weights share the launch),
// otherwise none is.
int gemm_q4k_sp_splits(int64_t n, int64_t k, int64_t rows, int cus);
size_t gemm_q4k_sp_split_bytes(const MvTargets& t, int64_t k, int64_t rows, int cus);
hipError_t launch_gemm_q4k_sp_targets(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, void* split_ws,
                                      size_t split_bytes, int cus, hipStream_t st);
// The same single-pass GEMM for Q6_K weights (k a multiple of 2048, from
// gemm_q4k_sp_min_rows() rows): w8 = round(m_j (q - 32) / 256) with
// m_j = round(127 sc_j / 16); same tiles, K splits and launches.
bool gemm_q6k_sp_fits(int64_t n, int64_t k, int64_t rows);
hipError_t launch_gemm_q6k_sp(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                              int64_t ldd, hipStream_t s);
hipError_t launch_gemm_q6k_sp_targets(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, void* split_ws,
                                      size_t split_bytes, int cus, hipStream_t st);

int gemm_q4k_min_rows();
// The GEMM indexes with 32-bit byte offsets: the weight below 2 GiB and
// (rows + 128) * k below 2^31.
bool gemm_q4k_fits(int64_t n, int64_t k, int64_t rows);
hipError_t launch_gemm_q4k(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                           int64_t ldd, hipStream_t s);

// The Q8_0 / IQ4_NL / MXFP4 GEMM (gemm_b32.hip), from gemm_b32_min_rows()
// rows: exact int32 block sums, f32 scaling per block.
int gemm_b32_min_rows();
bool gemm_b32_fits(int type, int64_t n, int64_t k, int64_t rows);
hipError_t launch_gemm_b32(int type, const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows,
                           float* dst, int64_t ldd, hipStream_t s);

// The Q6_K GEMM (gemm_q6k.hip), from gemm_q6k_min_rows() rows, exact int32
// super-block sums; the same 32-bit offset limits.
int gemm_q6k_min_rows();
bool gemm_q6k_fits(int64_t n, int64_t k, int64_t rows);
hipError_t launch_gemm_q6k(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                           int64_t ldd, hipStream_t s);

// Set-up a first launch would otherwise do (qmm_prepare): the LDS limit of
// every kernel that asks for more than 64 KiB, on the current device, and
// the no-allocation scratch's address there.
hipError_t raise_all_lds_limits();

// SWARMLLM_QMATMUL_EXACT (read once): only the exact Q4_K / Q6_K forms.
bool exact_forms();
bool noalloc_prepare();

}  // namespace qmm
