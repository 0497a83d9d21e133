// moe.hip — grouped expert products for the 32-value formats (MXFP4, Q8_0,
// IQ4_NL) on gfx950: the work of candle-kernels' moe_gemm_gguf
// (vendor/candle/candle-kernels/src/moe/moe_gguf.cu:149-252, called from
// src/layers/moe_card.rs:48-170) and of QMatMul::matmul_many over the
// touched experts (vendor/candle/candle-core/src/quantized/mod.rs:697-780).
//
// Entry i of the routing (i < size_m) is the pair p = sorted_ids[i] (a
// token's k-th choice, numbered token * topk + k) and its expert
// e = expert_ids[i]. It computes
//     dst[p][j] = scale_p * (x[in_p] . W_e[j])   for weight rows j < n
// with in_p = p (per-pair inputs, topk_w given) or p / topk (per-token
// inputs), scale_p = topk_w[p] or 1, the activation quantized per 32 values
// (Q8_0, the VecDotType of these formats). An entry whose expert or pair is
// out of range writes nothing, as in the reference.
//
// Shape of the work: a pre-pass (moe_runs_kernel, one workgroup) cuts the
// routing into runs of consecutive entries with the same expert — with ids
// sorted by expert, one run per touched expert — so the products of a run
// read the expert's weights once: a wave stages each weight row's blocks in
// LDS and applies them to up to 8 of the run's activation rows at a time.
// The per-unit arithmetic and the reduction are the decode kernel's
// (b32_common.h, wave_sum_dpp), so each pair's result is bit-identical to
// the same product through qmm_forward (times its scale): the reference's
// "matmul_many equals per-job forward" (quantized/mod.rs:743-745).
#include "b32_common.h"

namespace qmm {

namespace {

constexpr int kMoeWaves = 4;   // waves per workgroup
constexpr int kMoePairs = 8;   // activation rows a wave applies a staged row to

// runs[0] = number of runs; run r at runs[1 + 3r]: first entry, length, expert.
__global__ __launch_bounds__(1024) void moe_runs_kernel(const int32_t* __restrict__ expert_ids, int size_m,
                                                        int32_t* __restrict__ runs) {
  __shared__ int32_t scan[1024];
  __shared__ int32_t base;
  const int t = threadIdx.x;
  if (t == 0) base = 0;
  __syncthreads();
  for (int c0 = 0; c0 < size_m; c0 += 1024) {
    const int i = c0 + t;
    const int e = i < size_m ? expert_ids[i] : 0;
    const int f = (i < size_m && (i == 0 || expert_ids[i - 1] != e)) ? 1 : 0;
    scan[t] = f;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {  // inclusive scan of the run-start flags
      const int v = t >= d ? scan[t - d] : 0;
      __syncthreads();
      scan[t] += v;
      __syncthreads();
    }
    if (f) {
      const int r = base + scan[t] - 1;
      runs[1 + 3 * r] = i;
      runs[3 + 3 * r] = e;
    }
    __syncthreads();
    if (t == 0) base += scan[1023];
    __syncthreads();
  }
  const int nr = base;
  for (int r = t; r < nr; r += 1024) {
    const int s = runs[1 + 3 * r];
    const int s2 = r + 1 < nr ? runs[1 + 3 * (r + 1)] : size_m;
    runs[2 + 3 * r] = s2 - s;
  }
  if (t == 0) runs[0] = nr;
}

template <int FMT, int RPW>
__global__ __launch_bounds__(64 * kMoeWaves) void moe_b32_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int32_t* __restrict__ runs,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m,
    float* __restrict__ dst, int64_t ldd) {
  using F = Fmt32<FMT>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kMoeWaves][RPW][kStageBytes];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row0 = ((int64_t)blockIdx.x * kMoeWaves + wv) * RPW;
  if (row0 >= n) return;  // waves sync only with themselves
  const int64_t k = (int64_t)nb * 32;
  const int64_t rb = (int64_t)nb * F::B;
  const Lut32<FMT> lut;
  const int nruns = __builtin_amdgcn_readfirstlane(runs[0]);

  for (int run = blockIdx.y; run < nruns; run += gridDim.y) {
    const int start = __builtin_amdgcn_readfirstlane(runs[1 + 3 * run]);
    const int len = __builtin_amdgcn_readfirstlane(runs[2 + 3 * run]);
    const int e = __builtin_amdgcn_readfirstlane(runs[3 + 3 * run]);
    if (e < 0 || e >= num_experts) continue;
    const uint8_t* We = W + (int64_t)e * estride;
    for (int c0 = 0; c0 < len; c0 += kMoePairs) {
      const int cnt = len - c0 < kMoePairs ? len - c0 : kMoePairs;
      int64_t in_row[kMoePairs];
      int64_t out_row[kMoePairs];
      float scale[kMoePairs];
      bool use[kMoePairs];
#pragma unroll
      for (int p = 0; p < kMoePairs; p++) {
        const int pair = p < cnt ? __builtin_amdgcn_readfirstlane(ids[start + c0 + p]) : -1;
        use[p] = pair >= 0 && pair < size_m;
        out_row[p] = use[p] ? pair : 0;
        in_row[p] = use[p] ? (topk_w ? pair : pair / topk) : 0;
        scale[p] = use[p] && topk_w ? topk_w[pair] : 1.0f;
      }
      float acc[kMoePairs][RPW];
#pragma unroll
      for (int p = 0; p < kMoePairs; p++)
#pragma unroll
        for (int i = 0; i < RPW; i++) acc[p][i] = 0.0f;

      for (int b0 = 0; b0 < nb; b0 += 128) {
        const int nspan = nb - b0 < 128 ? nb - b0 : 128;
        int off[RPW];
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < RPW; i++) {
          const int64_t row = row0 + i < n ? row0 + i : n - 1;
          off[i] = stage_span(We, row * rb + (int64_t)b0 * F::B, nspan * F::B, smem[wv][i], lane);
        }
        wave_lds_sync();
        const int bl = 2 * lane;  // first block of this lane's unit, within the span
        if (bl < nspan) {
          const bool two = bl + 1 < nspan;
          uint32_t q[RPW][2][8];
          float dx[RPW][2];
#pragma unroll
          for (int i = 0; i < RPW; i++) {
            F::decode(smem[wv][i], off[i] + bl * F::B, q[i][0], dx[i][0], lut.t0, lut.t1, lut.t2, lut.t3);
            if (two) {
              F::decode(smem[wv][i], off[i] + (bl + 1) * F::B, q[i][1], dx[i][1], lut.t0, lut.t1, lut.t2, lut.t3);
            } else {
#pragma unroll
              for (int t = 0; t < 8; t++) q[i][1][t] = 0;
              dx[i][1] = 0.0f;
            }
          }
          const int64_t gb = b0 + bl;
#pragma unroll
          for (int p = 0; p < kMoePairs; p++) {
            if (!use[p]) continue;
            Act64 av;
            load_act64(av, yq, yd, in_row[p], k, nb, gb, two);
#pragma unroll
            for (int i = 0; i < RPW; i++) acc[p][i] = b32_unit(q[i][0], q[i][1], dx[i][0], dx[i][1], av, acc[p][i]);
          }
        }
      }
#pragma unroll
      for (int p = 0; p < kMoePairs; p++) {
        if (!use[p]) continue;
#pragma unroll
        for (int i = 0; i < RPW; i++) {
          const float v = wave_sum_dpp(acc[p][i]);
          if (lane == 0 && row0 + i < n) dst[out_row[p] * ldd + row0 + i] = __fmul_rn(v, scale[p]);
        }
      }
    }
  }
}

template <int FMT>
hipError_t launch_moe_fmt(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                          const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                          float* dst, int64_t ldd, hipStream_t st) {
  constexpr int RPW = 2;
  const int nb = (int)(k / 32);
  const int64_t estride = n * nb * Fmt32<FMT>::B;
  const int64_t waves = (n + RPW - 1) / RPW;
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  const dim3 grid((unsigned)((waves + kMoeWaves - 1) / kMoeWaves), (unsigned)(gy < 1 ? 1 : gy));
  moe_b32_kernel<FMT, RPW><<<grid, 64 * kMoeWaves, 0, st>>>((const uint8_t*)w, n, nb, estride, num_experts, p.codes,
                                                           p.d, runs, ids, topk_w, topk, (int)size_m, dst, ldd);
  return hipGetLastError();
}

}  // namespace

bool moe_supported(int type) { return type == T_Q8_0 || type == T_IQ4_NL || type == T_MXFP4; }

size_t moe_runs_bytes(int64_t size_m) { return (size_t)(1 + 3 * size_m) * sizeof(int32_t); }

hipError_t launch_moe(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                      int32_t* runs, const int32_t* ids, const int32_t* expert_ids, const float* topk_w, int topk,
                      int64_t size_m, float* dst, int64_t ldd, hipStream_t st) {
  moe_runs_kernel<<<1, 1024, 0, st>>>(expert_ids, (int)size_m, runs);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (type) {
    case T_Q8_0: return launch_moe_fmt<T_Q8_0>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
    case T_IQ4_NL:
      return launch_moe_fmt<T_IQ4_NL>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
    case T_MXFP4:
      return launch_moe_fmt<T_MXFP4>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qmm
