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

}  // namespace qmm
