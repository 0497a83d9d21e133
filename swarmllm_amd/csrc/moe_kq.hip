// moe_kq.hip — grouped expert products for the K-quant formats (Q4_K, Q6_K)
// on gfx950: the work of candle-kernels' moe_gemm_gguf for these weight types
// (vendor/candle/candle-kernels/src/moe/moe_gguf.cu:149-252, its FFI at
// vendor/candle/candle-kernels/src/ffi.rs:24-37; called from
// src/layers/moe_card.rs:48-170) and of QMatMul::matmul_many over the touched
// experts (vendor/candle/candle-core/src/quantized/mod.rs:697-780).
//
// Entry i of the routing (i < size_m) pairs p = sorted_ids[i] with expert
// e = expert_ids[i] and computes
//     dst[p][j] = scale_p * (x[in_p] . W_e[j])   for weight rows j < n
// with in_p = p (per-pair inputs, topk_w given) or p / topk, scale_p =
// topk_w[p] or 1, the activation quantized per 256 values (Q8_K, the
// VecDotType of both formats). An entry whose expert or pair is out of range
// writes nothing.
//
// Shape of the work: as the 32-value grouped kernel (moe.hip). The routing is
// cut into runs of consecutive entries with the same expert (moe_runs.h); a
// workgroup takes one run and a block of the expert's rows, copies the
// quantized activation rows of a chunk of the run's entries into LDS, and
// each wave walks its weight rows, applying each to every entry of the chunk.
//
// Per entry the lane-to-unit mapping, the unit arithmetic (q4k_unit,
// q6k_unit) and the order of the sums are those of the 1-row decode kernels
// (mv_q4k.hip: a lane's units of super-blocks L/4 + 16t summed over t, then
// one wave reduction; mv_q6k.hip: spans of 16 super-blocks, a wave reduction
// per span, the spans' sums added in order), so each entry's result is
// bit-identical to qmm_forward of its input row, times its scale: the
// reference's "matmul_many equals per-job forward"
// (quantized/mod.rs:743-745).
#include "mv_common.h"

namespace qmm {

namespace {

constexpr int kKqWaves = 8;  // waves per workgroup
constexpr int kKqPairs = 8;  // most entries a chunk holds
constexpr size_t kKqLdsBudget = 64 * 1024;

// The chunk's activation rows in LDS: codes int8 [P][k], group sums int16
// [P][nsb*16], scales f32 [P][nsb]; then (Q6_K) a span buffer per wave.
__host__ __device__ inline size_t kq_pair_bytes(int nsb) { return (size_t)nsb * (256 + 32 + 4); }
__host__ __device__ inline size_t kq_act_bytes(int nsb, int pairs) {
  return ((size_t)pairs * kq_pair_bytes(nsb) + 15) / 16 * 16;
}

template <int TYPE>
__host__ __device__ inline size_t kq_stage_bytes() {
  return TYPE == T_Q6_K ? (size_t)kKqWaves * kQ6SpanBuf : 0;
}

// Q4_K: the header and the lane's 32 code bytes of each of its super-blocks
// sbl + 16t of a row (mv_q4k.hip's per-lane layout).
template <int T>
struct Q4Row {
  uint4 h[T], qa[T], qb[T];
};

template <int T>
__device__ __forceinline__ void load_q4_row(Q4Row<T>& rr, const uint8_t* __restrict__ row, int nsb, int j, int sbl) {
#pragma unroll
  for (int t = 0; t < T; t++) {
    const int sb = sbl + 16 * t;
    const uint8_t* blk = row + 144 * (sb < nsb ? sb : nsb - 1);
    rr.h[t] = ld_stream16(blk);
    rr.qa[t] = ld_stream16(blk + 16 + 32 * j);
    rr.qb[t] = ld_stream16(blk + 32 + 32 * j);
  }
}

template <int TYPE, int T>
__global__ __launch_bounds__(64 * kKqWaves) void moe_kq_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nsb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int16_t* __restrict__ ybs,
    const int32_t* __restrict__ runs, const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk,
    int size_m, float* __restrict__ dst, int64_t ldd, int rpw, int npairs) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int k = nsb * 256;
  int8_t* const acodes = (int8_t*)smem;                                     // [P][k]
  int16_t* const asums = (int16_t*)(smem + (size_t)npairs * k);             // [P][nsb*16]
  float* const ad = (float*)(smem + (size_t)npairs * (k + 32 * nsb));       // [P][nsb]
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + kq_act_bytes(nsb, npairs) + (size_t)wv * kQ6SpanBuf;  // Q6_K only

  const int64_t rowbytes = (int64_t)nsb * (TYPE == T_Q4_K ? 144 : 210);
  const int64_t r0 = ((int64_t)blockIdx.x * kKqWaves + wv) * rpw;
  const int nrows = r0 < n ? (int)(n - r0 < rpw ? n - r0 : rpw) : 0;
  // Q4_K lanes: chunk j of super-blocks sbl + 16t; Q6_K lanes: unit u of
  // super-block sbl of a span (half h, l0)
  const int j = lane & 3, sbl = lane >> 2, h = j >> 1, l0 = 16 * (j & 1);
  const int nspan = (nsb + kQ6SpanSb - 1) / kQ6SpanSb;

  // Runs blockIdx.y, blockIdx.y + gridDim.y, ...; the loop and its barriers
  // are uniform over the workgroup.
  const int nruns = __builtin_amdgcn_readfirstlane(runs[0]);
  for (int run = blockIdx.y; run < nruns; run += gridDim.y) {
    const int start = __builtin_amdgcn_readfirstlane(runs[1 + 3 * run]);
    const int len = __builtin_amdgcn_readfirstlane(runs[2 + 3 * run]);
    const int e = __builtin_amdgcn_readfirstlane(runs[3 + 3 * run]);
    if (e < 0 || e >= num_experts) continue;
    const uint8_t* We = W + (int64_t)e * estride;

    for (int c0 = 0; c0 < len; c0 += npairs) {
      const int cnt = len - c0 < npairs ? len - c0 : npairs;
      int pr[kKqPairs];
#pragma unroll
      for (int p = 0; p < kKqPairs; p++)
        pr[p] = __builtin_amdgcn_readfirstlane(ids[start + c0 + (p < cnt ? p : cnt - 1)]);
      bool use[kKqPairs];
      int64_t out_row[kKqPairs], in_row[kKqPairs];
      float scale[kKqPairs];
#pragma unroll
      for (int p = 0; p < kKqPairs; p++) {
        use[p] = p < cnt && pr[p] >= 0 && pr[p] < size_m;
        out_row[p] = use[p] ? pr[p] : 0;
        in_row[p] = use[p] ? (topk_w ? pr[p] : pr[p] / topk) : 0;
        scale[p] = topk_w ? topk_w[use[p] ? pr[p] : 0] : 1.0f;
      }

      // the chunk's activation rows into LDS, after the previous chunk's reads
      __syncthreads();
      {
        const int cpr = k / 16, spr = 2 * nsb;  // 16-byte pieces a row: codes, group sums
#pragma unroll
        for (int p = 0; p < kKqPairs; p++) {
          if (!use[p]) continue;
          const int8_t* cr = yq + in_row[p] * k;
          const int16_t* sr = ybs + in_row[p] * (16 * nsb);
          const float* dr = yd + in_row[p] * nsb;
          for (int i = threadIdx.x; i < cpr; i += 64 * kKqWaves)
            *(uint4*)(acodes + (size_t)p * k + 16 * i) = *(const uint4*)(cr + 16 * i);
          for (int i = threadIdx.x; i < spr; i += 64 * kKqWaves)
            *(uint4*)(asums + (size_t)p * 16 * nsb + 8 * i) = *(const uint4*)(sr + 8 * i);
          for (int i = threadIdx.x; i < nsb; i += 64 * kKqWaves) ad[p * nsb + i] = dr[i];
        }
      }
      __syncthreads();

      if constexpr (TYPE == T_Q4_K) {
        // rows in order, the next row's loads in flight under this row's units
        Q4Row<T> cur, nxt;
        if (nrows > 0) load_q4_row<T>(cur, We + r0 * rowbytes, nsb, j, sbl);
        for (int i = 0; i < nrows; i++) {
          if (i + 1 < nrows) load_q4_row<T>(nxt, We + (r0 + i + 1) * rowbytes, nsb, j, sbl);
          float acc[kKqPairs];
#pragma unroll
          for (int p = 0; p < kKqPairs; p++) acc[p] = 0.0f;
#pragma unroll
          for (int t = 0; t < T; t++) {
            const int sb = sbl + 16 * t;
            if (sb < nsb) {
#pragma unroll
              for (int p = 0; p < kKqPairs; p++) {
                if (!use[p]) continue;
                const int4* yp = (const int4*)(acodes + p * k + sb * 256 + 64 * j);
                int y[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                  const int4 v = yp[q];
                  y[4 * q] = v.x; y[4 * q + 1] = v.y; y[4 * q + 2] = v.z; y[4 * q + 3] = v.w;
                }
                // sub-blocks 2j, 2j+1 = groups 4j .. 4j+3
                const uint2 g = *(const uint2*)(asums + (p * nsb + sb) * 16 + 4 * j);
                const int32_t p0 = (int32_t)(int16_t)(g.x & 0xFFFF) + (int32_t)(int16_t)(g.x >> 16);
                const int32_t p1 = (int32_t)(int16_t)(g.y & 0xFFFF) + (int32_t)(int16_t)(g.y >> 16);
                acc[p] = q4k_unit(cur.h[t], cur.qa[t], cur.qb[t], y, ad[p * nsb + sb], p0, p1, j, acc[p]);
              }
            }
          }
#pragma unroll
          for (int p = 0; p < kKqPairs; p++) {
            if (!use[p]) continue;
            const float v = wave_sum_dpp(acc[p]);
            if (lane == 0) dst[out_row[p] * ldd + r0 + i] = __fmul_rn(v, scale[p]);
          }
          cur = nxt;
        }
      } else {
        // spans of 16 super-blocks in order, the next span's loads in flight;
        // past the wave's last span the loads read the (cached) first bytes
        // of the quantized activation, never used
        const int S = nrows * nspan;
        int lr = 0, lsp = 0;  // the span loaded next: span lsp of row r0 + lr
        auto load_next = [&](Q6Span& spn) {
          if (lr < nrows) {
            const int s0 = lsp * kQ6SpanSb;
            load_q6_span(spn, We + (r0 + lr) * rowbytes + (int64_t)s0 * 210, nsb - s0 < kQ6SpanSb ? nsb - s0 : kQ6SpanSb,
                         lane);
          } else {
            load_q6_span(spn, (const uint8_t*)yq, 1, lane);
          }
          if (++lsp == nspan) {
            lsp = 0;
            lr++;
          }
        };
        Q6Span cur;
        load_next(cur);
        float tot[kKqPairs];
#pragma unroll
        for (int p = 0; p < kKqPairs; p++) tot[p] = 0.0f;
        int row = 0, sp = 0;
        for (int s = 0; s < S; s++) {
          wave_lds_sync();
#pragma unroll
          for (int c = 0; c < kQ6PiecesPerLane; c++) {
            const int pc = lane + 64 * c;
            *(uint4*)(buf + 16 * (pc < kQ6SpanPieces ? pc : kQ6SpanPieces - 1)) = cur.p[c];
          }
          wave_lds_sync();
          const int off = cur.off, slen = cur.len;
          load_next(cur);
          float acc[kKqPairs];
#pragma unroll
          for (int p = 0; p < kKqPairs; p++) acc[p] = 0.0f;
          if (sbl < slen) {
            Q6Lane u;
            load_q6_lane(buf, off + 210 * sbl, h, l0, u);
            const int sb = sp * kQ6SpanSb + sbl;
#pragma unroll
            for (int p = 0; p < kKqPairs; p++) {
              if (!use[p]) continue;
              const int8_t* yrow = acodes + p * k + sb * 256 + 128 * h + l0;
              int yv[4][4], bs[4];
#pragma unroll
              for (int t = 0; t < 4; t++) {
                const int4 q = *(const int4*)(yrow + 32 * t);
                yv[t][0] = q.x; yv[t][1] = q.y; yv[t][2] = q.z; yv[t][3] = q.w;
                bs[t] = asums[(p * nsb + sb) * 16 + 8 * h + 2 * t + (l0 >> 4)];
              }
              acc[p] = q6k_unit(u.qlA, u.qlB, u.qh, u.sc, u.dx, yv, ad[p * nsb + sb], bs, acc[p]);
            }
          }
          // the span's sum, added to its row's in span order
#pragma unroll
          for (int p = 0; p < kKqPairs; p++) {
            if (!use[p]) continue;
            const float v = wave_sum_dpp(acc[p]);
            tot[p] = sp == 0 ? v : __fadd_rn(tot[p], v);
          }
          if (++sp == nspan) {
#pragma unroll
            for (int p = 0; p < kKqPairs; p++)
              if (use[p] && lane == 0) dst[out_row[p] * ldd + r0 + row] = __fmul_rn(tot[p], scale[p]);
            sp = 0;
            row++;
          }
        }
      }
    }
  }
}

template <int TYPE, int T>
hipError_t launch_kq(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p, const int32_t* runs,
                     const int32_t* ids, const float* topk_w, int topk, int64_t size_m, float* dst, int64_t ldd,
                     int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int nsb = (int)(k / 256);
  const int64_t estride = n * nsb * (TYPE == T_Q4_K ? 144 : 210);
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  // entries a chunk: as many as the LDS budget holds, up to kKqPairs
  int64_t pairs = (int64_t)((kKqLdsBudget - kq_stage_bytes<TYPE>()) / kq_pair_bytes(nsb));
  if (pairs > kKqPairs) pairs = kKqPairs;
  if (pairs < 1) pairs = 1;
  // rows a wave: one while the runs' rows fill 32 waves a CU, more beyond
  int64_t rpw = (n * gy + (int64_t)cus * 32 - 1) / ((int64_t)cus * 32);
  if (rpw < 1) rpw = 1;
  if (rpw > 64) rpw = 64;
  const int64_t rows_per_wg = (int64_t)kKqWaves * rpw;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = kq_act_bytes(nsb, (int)pairs) + kq_stage_bytes<TYPE>();
  auto* kfn = &moe_kq_kernel<TYPE, T>;
  if (lds > 65536 && set_max_dynamic_lds((const void*)kfn) != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kKqWaves, lds, st>>>((const uint8_t*)w, n, nsb, estride, num_experts, p.codes, p.d,
                                        (const int16_t*)p.sums, runs, ids, topk_w, topk, (int)size_m, dst, ldd,
                                        (int)rpw, (int)pairs);
  return hipGetLastError();
}

}  // namespace

// Rows of up to 16384 values, where both 1-row decode kernels (whose sums
// these kernels reproduce) take the product and a chunk's activation row fits
// the LDS budget beside the span buffers.
bool moe_kq_supported(int type, int64_t k) {
  return (type == T_Q4_K || type == T_Q6_K) && k % 256 == 0 && k >= 256 && k <= 16384;
}

hipError_t launch_moe_kq(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                         const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                         float* dst, int64_t ldd, int cus, hipStream_t st) {
  if (!moe_kq_supported(type, k)) return hipErrorInvalidValue;
  if (type == T_Q6_K)
    return launch_kq<T_Q6_K, 1>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
  const int T = (int)((k / 256 + 15) / 16);
  if (T <= 1) return launch_kq<T_Q4_K, 1>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
  if (T <= 2) return launch_kq<T_Q4_K, 2>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
  return launch_kq<T_Q4_K, 4>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
}

}  // namespace qmm
