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

// Entries go through in blocks of NT x kRunsPer: each thread loads its
// kRunsPer consecutive ids (and the one before) at once, counts the run
// starts among them, and one scan over the block numbers them, so a routing
// of size_m entries costs size_m / (NT kRunsPer) dependent rounds.
constexpr int kRunsPer = 8;

template <int NT>
__device__ __forceinline__ void moe_runs_block(const int32_t* __restrict__ expert_ids, int size_m,
                                               int32_t* __restrict__ runs) {
  static_assert(NT % 64 == 0 && NT <= 1024, "whole waves");
  constexpr int kW = NT / 64;
  __shared__ int s_cnt[kW];
  const int t = (int)threadIdx.x, lane = t & 63, w = t >> 6;
  int base = 0;  // runs started before this block
  for (int c0 = 0; c0 < size_m; c0 += NT * kRunsPer) {
    const int i0 = c0 + t * kRunsPer;
    int id[kRunsPer];
#pragma unroll
    for (int j = 0; j < kRunsPer; j++) id[j] = i0 + j < size_m ? expert_ids[i0 + j] : 0;
    int prev = i0 > 0 && i0 <= size_m ? expert_ids[i0 - 1] : 0;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kRunsPer; j++) {
      cnt += (i0 + j < size_m && (i0 + j == 0 || id[j] != prev)) ? 1 : 0;
      prev = id[j];
    }
    int v = cnt;  // inclusive sum over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int u = __shfl_up(v, d);
      if (lane >= d) v += u;
    }
    if (lane == 63) s_cnt[w] = v;
    __syncthreads();
    int before = base, total = base;
#pragma unroll
    for (int j = 0; j < kW; j++) {
      const int c = s_cnt[j];
      before += j < w ? c : 0;
      total += c;
    }
    // this thread's starts are numbered from before + (the wave's lanes below)
    int r = before + v - cnt;
    prev = i0 > 0 && i0 <= size_m ? expert_ids[i0 - 1] : 0;
#pragma unroll
    for (int j = 0; j < kRunsPer; j++) {
      if (i0 + j < size_m && (i0 + j == 0 || id[j] != prev)) {
        runs[1 + 3 * r] = i0 + j;
        runs[3 + 3 * r] = id[j];
        r++;
      }
      prev = id[j];
    }
    base = total;
    __syncthreads();  // s_cnt is rewritten by the next block
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
