// moe_runs.h — the run table of a grouped expert product, written by one
// workgroup of NT threads.
//
// The routing's entries i < size_m pair sorted_ids[i] with expert_ids[i]. A
// run is a maximal stretch of consecutive entries with the same expert: it
// starts at entry 0 and wherever the expert differs from the entry before
// (with entries grouped by expert, one run per touched expert, the grouping
// moe_gemm_gguf's callers produce, moe_card.rs:48-170). The table:
//   runs[0] = number of runs; run r at runs[1 + 3r]: first entry, length, expert.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace qmm {

template <int NT>
__device__ __forceinline__ void moe_runs_block(const int32_t* __restrict__ expert_ids, int size_m,
                                               int32_t* __restrict__ runs) {
  static_assert(NT % 64 == 0 && NT <= 1024, "whole waves");
  constexpr int kW = NT / 64;
  __shared__ int s_cnt[kW];
  const int t = (int)threadIdx.x, lane = t & 63, w = t >> 6;
  int base = 0;  // runs started before this chunk
  for (int c0 = 0; c0 < size_m; c0 += NT) {
    const int i = c0 + t;
    const bool in = i < size_m;
    const int e = in ? expert_ids[i] : 0;
    const bool f = in && (i == 0 || expert_ids[i - 1] != e);
    const uint64_t m = __ballot(f);
    if (lane == 0) s_cnt[w] = __popcll(m);
    __syncthreads();
    int before = base, total = base;
#pragma unroll
    for (int j = 0; j < kW; j++) {
      const int c = s_cnt[j];
      before += j < w ? c : 0;
      total += c;
    }
    if (f) {
      // this start's number: the chunk's earlier waves' starts, then this wave's below this lane
      const int r = before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      runs[1 + 3 * r] = i;
      runs[3 + 3 * r] = e;
    }
    base = total;
    __syncthreads();  // s_cnt is rewritten by the next chunk
  }
  // the starts are written (the barrier orders the workgroup's global
  // writes before these reads); run r ends where run r + 1 starts
  for (int r = t; r < base; r += NT) {
    const int s = runs[1 + 3 * r];
    const int s2 = r + 1 < base ? runs[1 + 3 * (r + 1)] : size_m;
    runs[2 + 3 * r] = s2 - s;
  }
  if (t == 0) runs[0] = base;
}

// The chunk table of a run table written by this workgroup: run r cut into
// ceil(len / ch) chunks of up to ch consecutive entries, in run order.
//   chunks[0] = number of chunks; chunk c at chunks[1 + 3c]: first entry,
//   length, expert.
// At most size_m / ch + (number of runs) chunks.
template <int NT>
__device__ __forceinline__ void moe_chunks_block(const int32_t* __restrict__ runs, int ch,
                                                 int32_t* __restrict__ chunks) {
  constexpr int kW = NT / 64;
  __shared__ int s_sum[kW];
  const int t = (int)threadIdx.x, lane = t & 63, w = t >> 6;
  __syncthreads();  // the run table is written
  const int nruns = runs[0];
  int base = 0;  // chunks of the runs before this block of runs
  for (int r0 = 0; r0 < nruns; r0 += NT) {
    const int r = r0 + t;
    const int len = r < nruns ? runs[2 + 3 * r] : 0;
    const int nc = (len + ch - 1) / ch;
    int v = nc;  // inclusive sum over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int u = __shfl_up(v, d);
      if (lane >= d) v += u;
    }
    if (lane == 63) s_sum[w] = v;
    __syncthreads();
    int before = base, total = base;
#pragma unroll
    for (int j = 0; j < kW; j++) {
      const int c = s_sum[j];
      before += j < w ? c : 0;
      total += c;
    }
    if (r < nruns) {
      const int first = before + v - nc, s = runs[1 + 3 * r], e = runs[3 + 3 * r];
      for (int c = 0; c < nc; c++) {
        chunks[1 + 3 * (first + c)] = s + c * ch;
        chunks[2 + 3 * (first + c)] = len - c * ch < ch ? len - c * ch : ch;
        chunks[3 + 3 * (first + c)] = e;
      }
    }
    base = total;
    __syncthreads();  // s_sum is rewritten by the next block of runs
  }
  if (t == 0) chunks[0] = base;
}

}  // namespace qmm
