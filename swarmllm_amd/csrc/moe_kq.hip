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
constexpr int kKqFusedMaxEntries = 256;  // routings the fused form takes (each wave scans them)
constexpr size_t kKqLdsBudget = 64 * 1024;

// The chunk's activation rows in LDS: codes int8 [P][k], group sums int16
// [P][nsb*16], scales f32 [P][nsb]; then (Q6_K) a span buffer per wave.
__host__ __device__ inline size_t kq_pair_bytes(int nsb) { return (size_t)nsb * (256 + 32 + 4); }
__host__ __device__ inline size_t kq_act_bytes(int nsb, int pairs) {
  return ((size_t)pairs * kq_pair_bytes(nsb) + 15) / 16 * 16;
}

template <int TYPE>
__host__ __device__ inline size_t kq_stage_bytes();

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

// Q6_K rows of up to 16 / P super-blocks, P rows a wave: lane group q (G =
// 64 / P lanes) stages row q's block span in its own slot of the wave's
// buffer, 4 aligned 16-byte pieces a lane.
template <int P>
struct Q6Pack {
  static constexpr int G = 64 / P;
  static constexpr int kSlot = G * 4 * 16;  // bytes a row: the pieces (the span and its over-read fit)
  uint4 p[4];
  int off;
};

template <int P>
__device__ __forceinline__ void load_q6_pack(Q6Pack<P>& sp, const uint8_t* __restrict__ row, int nsb, int pl) {
  sp.off = (int)((uintptr_t)row & 15);
  const uint8_t* a0 = row - sp.off;
  const int pieces = (sp.off + nsb * 210 + 15) >> 4;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int pc = pl + Q6Pack<P>::G * c;
    sp.p[c] = ld_stream16(a0 + 16u * (uint32_t)(pc < pieces ? pc : pieces - 1));
  }
}

// LDS bytes a wave stages Q6_K spans in
constexpr int kKqStageBuf = kQ6SpanBuf > 4 * 1024 + 16 ? kQ6SpanBuf : 4 * 1024 + 16;

template <int TYPE>
__host__ __device__ inline size_t kq_stage_bytes() {
  return TYPE == T_Q6_K ? (size_t)kKqWaves * kKqStageBuf : 0;
}

// P weight rows a wave at a time (P = 2, 4 where a row's units take at most
// 64 / P lanes: Q4_K and Q6_K rows of at most 8 or 4 super-blocks). Row q of
// the P takes lanes [q G, (q + 1) G) with the 1-row decode kernel's lane
// mapping inside them, and its sum is the 16-lane row sums of its lanes:
// the 1-row kernel's wave sum (a + b) + (c + d) over the same units, whose
// other rows of lanes hold no unit and add +0 (a sum of units is never -0:
// every lane's sum starts at +0), so each row's result is bit-identical.
// kFused: the kernel takes the f32 input rows and the routing's expert ids
// itself (the one launch of a small routing): each wave finds its runs in
// expert_ids, and the chunk's Q8_K codes, group sums and scales are made in
// LDS by q8k_block_group16, act_q8k_kernel's routine (quantize.hip), so they
// have its bits. Otherwise they come from launch_act_quantize_moe.
template <int TYPE, int T, int P, bool kFused>
__global__ __launch_bounds__(64 * kKqWaves) void moe_kq_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nsb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int16_t* __restrict__ ybs,
    const int32_t* __restrict__ runs, const float* __restrict__ xa, int64_t x_stride,
    const int32_t* __restrict__ expert_ids, int xvec, float qmax, const int32_t* __restrict__ ids,
    const float* __restrict__ topk_w, int topk, int size_m, float* __restrict__ dst, int64_t ldd, int rpw,
    int npairs) {
  static_assert(P == 1 || T == 1, "packed rows take one unit a lane");
  constexpr int G = 64 / P;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int k = nsb * 256;
  int8_t* const acodes = (int8_t*)smem;                                     // [P][k]
  int16_t* const asums = (int16_t*)(smem + (size_t)npairs * k);             // [P][nsb*16]
  float* const ad = (float*)(smem + (size_t)npairs * (k + 32 * nsb));       // [P][nsb]
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + kq_act_bytes(nsb, npairs) + (size_t)wv * kKqStageBuf;  // Q6_K only

  const int64_t rowbytes = (int64_t)nsb * (TYPE == T_Q4_K ? 144 : 210);
  const int64_t r0 = ((int64_t)blockIdx.x * kKqWaves + wv) * rpw;
  const int nrows = r0 < n ? (int)(n - r0 < rpw ? n - r0 : rpw) : 0;
  const int iters = (nrows + P - 1) / P;
  // the lane's row of a pack and its place in it: Q4_K chunk j of
  // super-blocks sbl + 16t; Q6_K unit (half h, l0) of super-block sbl of a span
  const int q = lane / G, pl = lane % G;
  const int j = pl & 3, sbl = pl >> 2, h = j >> 1, l0 = 16 * (j & 1);
  const int nspan = (nsb + kQ6SpanSb - 1) / kQ6SpanSb;
  // row of iteration it for this lane (the last row again past the wave's rows)
  auto prow = [&](int it) -> int64_t {
    const int r = it * P + q;
    return r0 + (r < nrows ? r : nrows - 1);
  };

  // Runs blockIdx.y, blockIdx.y + gridDim.y, ...; the loop and its barriers
  // are uniform over the workgroup.
  // fused: a run starts at entry 0 and wherever the expert differs from the
  // entry before (moe_runs_block's table, found by ballots over 64 entries)
  auto run_start = [&](int i) { return i < size_m && (i == 0 || expert_ids[i] != expert_ids[i - 1]); };
  int nruns;
  if (kFused) {
    int c = 0;
    for (int c0 = 0; c0 < size_m; c0 += 64) c += __builtin_popcountll(__ballot(run_start(c0 + lane)));
    nruns = __builtin_amdgcn_readfirstlane(c);
  } else {
    nruns = __builtin_amdgcn_readfirstlane(runs[0]);
  }
  for (int run = blockIdx.y; run < nruns; run += gridDim.y) {
    int start, len, e;
    if (kFused) {
      // the run-th and (run + 1)-th starts (size_m past the last)
      int s0 = size_m, s1 = size_m, cum = 0;
      for (int c0 = 0; c0 < size_m; c0 += 64) {
        const bool f = run_start(c0 + lane);
        const uint64_t m = __ballot(f);
        const int rank = cum + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        const uint64_t m0 = __ballot(f && rank == run), m1 = __ballot(f && rank == run + 1);
        if (m0 && s0 == size_m) s0 = c0 + __builtin_ctzll(m0);
        if (m1 && s1 == size_m) s1 = c0 + __builtin_ctzll(m1);
        cum += __builtin_popcountll(m);
      }
      start = __builtin_amdgcn_readfirstlane(s0);
      len = __builtin_amdgcn_readfirstlane(s1 - s0);
      e = __builtin_amdgcn_readfirstlane(expert_ids[start]);
    } else {
      start = __builtin_amdgcn_readfirstlane(runs[1 + 3 * run]);
      len = __builtin_amdgcn_readfirstlane(runs[2 + 3 * run]);
      e = __builtin_amdgcn_readfirstlane(runs[3 + 3 * run]);
    }
    if (e < 0 || e >= num_experts) continue;
    const uint8_t* We = W + (int64_t)e * estride;

    for (int c0 = 0; c0 < len; c0 += npairs) {
      const int cnt = len - c0 < npairs ? len - c0 : npairs;
      // the first rows' weight loads go out before the entries are looked up
      Q4Row<T> q4cur;
      Q6Pack<P> q6cur;
      Q6Span q6s;
      int lr = 0, lsp = 0;  // Q6_K, one row a wave: the span loaded next (span lsp of row r0 + lr)
      auto load_next = [&](Q6Span& spn) {
        if (lr < nrows) {
          const int s0 = lsp * kQ6SpanSb;
          load_q6_span(spn, We + (r0 + lr) * rowbytes + (int64_t)s0 * 210, nsb - s0 < kQ6SpanSb ? nsb - s0 : kQ6SpanSb,
                       lane);
        } else {
          load_q6_span(spn, We, 1, lane);  // (the expert's first super-block: cached, never used)
        }
        if (++lsp == nspan) {
          lsp = 0;
          lr++;
        }
      };
      if constexpr (TYPE == T_Q4_K) {
        if (nrows > 0) load_q4_row<T>(q4cur, We + prow(0) * rowbytes, nsb, j, sbl);
      } else if constexpr (P > 1) {
        if (nrows > 0) load_q6_pack<P>(q6cur, We + prow(0) * rowbytes, nsb, pl);
      } else {
        load_next(q6s);
      }

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
      if (kFused) {
        // 16 lanes a super-block of an entry's input row, as act_q8k_kernel
        const int gl = lane & 15;
        for (int t = threadIdx.x >> 4; t < npairs * nsb; t += 4 * kKqWaves) {
          const int p = t / nsb, b = t - p * nsb;  // uniform over the 16 lanes
          bool u = false;
          int64_t ir = 0;
#pragma unroll
          for (int pp = 0; pp < kKqPairs; pp++)
            if (p == pp) u = use[pp], ir = in_row[pp];
          if (!u) continue;
          const float* xp = xa + ir * x_stride + (int64_t)b * 256 + 16 * gl;
          float v[16];
          if (xvec) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const float4 f = ((const float4*)xp)[i];
              v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
            }
          } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = xp[i];
          }
          uint32_t c[4];
          int32_t sum16;
          float d;
          q8k_block_group16(v, gl, qmax, c, sum16, d);
          *(uint4*)(acodes + (size_t)p * k + 256 * b + 16 * gl) = make_uint4(c[0], c[1], c[2], c[3]);
          asums[(size_t)p * 16 * nsb + 16 * b + gl] = (int16_t)sum16;
          if (gl == 0) ad[p * nsb + b] = d;
        }
      } else {
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

      // a pack's sums per entry, stored by lane 0 (the results are wave-uniform)
      auto store = [&](int it, const float (&acc)[kKqPairs]) {
#pragma unroll
        for (int p = 0; p < kKqPairs; p++) {
          if (!use[p]) continue;
          float v[4];
          if constexpr (P == 1) {
            v[0] = wave_sum_dpp(acc[p]);
          } else {
            float a, b, c, d;
            wave_row16_sums(acc[p], a, b, c, d);
            if constexpr (P == 2) {
              v[0] = __fadd_rn(a, b);
              v[1] = __fadd_rn(c, d);
            } else {
              v[0] = a;
              v[1] = b;
              v[2] = c;
              v[3] = d;
            }
          }
          if (lane == 0) {
#pragma unroll
            for (int qq = 0; qq < P; qq++)
              if (it * P + qq < nrows) dst[out_row[p] * ldd + r0 + it * P + qq] = __fmul_rn(v[qq], scale[p]);
          }
        }
      };

      if constexpr (TYPE == T_Q4_K) {
        // rows in order, the next pack's loads in flight under this one's units
        Q4Row<T> nxt;
        for (int it = 0; it < iters; it++) {
          if (it + 1 < iters) load_q4_row<T>(nxt, We + prow(it + 1) * rowbytes, nsb, j, sbl);
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
                for (int qq = 0; qq < 4; qq++) {
                  const int4 v = yp[qq];
                  y[4 * qq] = v.x; y[4 * qq + 1] = v.y; y[4 * qq + 2] = v.z; y[4 * qq + 3] = v.w;
                }
                // sub-blocks 2j, 2j+1 = groups 4j .. 4j+3
                const uint2 g = *(const uint2*)(asums + (p * nsb + sb) * 16 + 4 * j);
                const int32_t p0 = (int32_t)(int16_t)(g.x & 0xFFFF) + (int32_t)(int16_t)(g.x >> 16);
                const int32_t p1 = (int32_t)(int16_t)(g.y & 0xFFFF) + (int32_t)(int16_t)(g.y >> 16);
                acc[p] = q4k_unit(q4cur.h[t], q4cur.qa[t], q4cur.qb[t], y, ad[p * nsb + sb], p0, p1, j, acc[p]);
              }
            }
          }
          store(it, acc);
          q4cur = nxt;
        }
      } else if constexpr (P > 1) {
        // packs of P rows, one span each, the next pack's loads in flight
        uint8_t* const slot = buf + q * Q6Pack<P>::kSlot;
        Q6Pack<P> nxt;
        for (int it = 0; it < iters; it++) {
          wave_lds_sync();
#pragma unroll
          for (int c = 0; c < 4; c++) *(uint4*)(slot + 16 * (pl + G * c)) = q6cur.p[c];
          wave_lds_sync();
          const int off = q6cur.off;
          if (it + 1 < iters) load_q6_pack<P>(nxt, We + prow(it + 1) * rowbytes, nsb, pl);
          float acc[kKqPairs];
#pragma unroll
          for (int p = 0; p < kKqPairs; p++) acc[p] = 0.0f;
          if (sbl < nsb) {
            Q6Lane u;
            load_q6_lane(slot, off + 210 * sbl, h, l0, u);
            const int sb = sbl;
#pragma unroll
            for (int p = 0; p < kKqPairs; p++) {
              if (!use[p]) continue;
              const int8_t* yrow = acodes + p * k + sb * 256 + 128 * h + l0;
              int yv[4][4], bs[4];
#pragma unroll
              for (int t = 0; t < 4; t++) {
                const int4 qv = *(const int4*)(yrow + 32 * t);
                yv[t][0] = qv.x; yv[t][1] = qv.y; yv[t][2] = qv.z; yv[t][3] = qv.w;
                bs[t] = asums[(p * nsb + sb) * 16 + 8 * h + 2 * t + (l0 >> 4)];
              }
              acc[p] = q6k_unit(u.qlA, u.qlB, u.qh, u.sc, u.dx, yv, ad[p * nsb + sb], bs, acc[p]);
            }
          }
          store(it, acc);
          q6cur = nxt;
        }
      } else {
        // spans of 16 super-blocks in order, the next span's loads in flight;
        // past the wave's last span the loads read the (cached) first bytes
        // of the quantized activation, never used
        const int S = nrows * nspan;
        float tot[kKqPairs];
#pragma unroll
        for (int p = 0; p < kKqPairs; p++) tot[p] = 0.0f;
        int row = 0, sp = 0;
        for (int sidx = 0; sidx < S; sidx++) {
          wave_lds_sync();
#pragma unroll
          for (int c = 0; c < kQ6PiecesPerLane; c++) {
            const int pc = lane + 64 * c;
            *(uint4*)(buf + 16 * (pc < kQ6SpanPieces ? pc : kQ6SpanPieces - 1)) = q6s.p[c];
          }
          wave_lds_sync();
          const int off = q6s.off, slen = q6s.len;
          load_next(q6s);
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
                const int4 qv = *(const int4*)(yrow + 32 * t);
                yv[t][0] = qv.x; yv[t][1] = qv.y; yv[t][2] = qv.z; yv[t][3] = qv.w;
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

// The fused form (fx set: the f32 input rows, expert ids, quantizer scale)
// or the form that reads launch_act_quantize_moe's planes and run table.
struct KqFused {
  const float* x;
  int64_t x_stride;
  const int32_t* expert_ids;
  float qmax;
};

template <int TYPE, int T, int P, bool kFused = false>
hipError_t launch_kq(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p, const int32_t* runs,
                     const int32_t* ids, const float* topk_w, int topk, int64_t size_m, float* dst, int64_t ldd,
                     int cus, hipStream_t st, const KqFused& fx = KqFused{}) {
  QMM_NOTE_LAUNCH();
  const int nsb = (int)(k / 256);
  const int64_t estride = n * nsb * (TYPE == T_Q4_K ? 144 : 210);
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  // entries a chunk: as many as the LDS budget holds, up to kKqPairs
  int64_t pairs = (int64_t)((kKqLdsBudget - kq_stage_bytes<TYPE>()) / kq_pair_bytes(nsb));
  if (pairs > kKqPairs) pairs = kKqPairs;
  if (pairs < 1) pairs = 1;
  // rows a wave: P while the runs' row packs fill 32 waves a CU, more beyond
  int64_t rpw = (n * gy + (int64_t)cus * 32 * P - 1) / ((int64_t)cus * 32 * P) * P;
  if (rpw < P) rpw = P;
  if (rpw > 64) rpw = 64;
  const int64_t rows_per_wg = (int64_t)kKqWaves * rpw;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = kq_act_bytes(nsb, (int)pairs) + kq_stage_bytes<TYPE>();
  constexpr auto* kfn = &moe_kq_kernel<TYPE, T, P, kFused>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  const int xvec = ((uintptr_t)fx.x % 16 == 0) && (fx.x_stride % 4 == 0);
  kfn<<<grid, 64 * kKqWaves, lds, st>>>((const uint8_t*)w, n, nsb, estride, num_experts, p.codes, p.d,
                                        (const int16_t*)p.sums, runs, fx.x, fx.x_stride, fx.expert_ids, xvec, fx.qmax,
                                        ids, topk_w, topk, (int)size_m, dst, ldd, (int)rpw, (int)pairs);
  return hipGetLastError();
}

template <bool kFused>
hipError_t launch_moe_kq_form(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                              const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                              float* dst, int64_t ldd, int cus, hipStream_t st, const KqFused& fx) {
  if (!moe_kq_supported(type, k)) return hipErrorInvalidValue;
  const int64_t nsb = k / 256;
#define KQ(TY, T, P) launch_kq<TY, T, P, kFused>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st, fx)
  if (type == T_Q6_K) {
    if (nsb <= 4) return KQ(T_Q6_K, 1, 4);
    if (nsb <= 8) return KQ(T_Q6_K, 1, 2);
    return KQ(T_Q6_K, 1, 1);
  }
  if (nsb <= 4) return KQ(T_Q4_K, 1, 4);
  if (nsb <= 8) return KQ(T_Q4_K, 1, 2);
  const int64_t T = (nsb + 15) / 16;
  if (T <= 1) return KQ(T_Q4_K, 1, 1);
  if (T <= 2) return KQ(T_Q4_K, 2, 1);
  return KQ(T_Q4_K, 4, 1);
#undef KQ
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
  return launch_moe_kq_form<false>(type, w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st,
                                   KqFused{});
}

bool moe_kq_fused_takes(int type, int64_t k, int64_t size_m) {
  return moe_kq_supported(type, k) && size_m <= kKqFusedMaxEntries;
}

hipError_t launch_moe_kq_fused(int type, const void* w, int num_experts, int64_t n, int64_t k, const float* x,
                               int64_t x_stride, const int32_t* expert_ids, const int32_t* ids, const float* topk_w,
                               int topk, int64_t size_m, float* dst, int64_t ldd, float qmax, int cus,
                               hipStream_t st) {
  return launch_moe_kq_form<true>(type, w, num_experts, n, k, ActPlanes{}, nullptr, ids, topk_w, topk, size_m, dst,
                                  ldd, cus, st, KqFused{x, x_stride, expert_ids, qmax});
}

}  // namespace qmm
