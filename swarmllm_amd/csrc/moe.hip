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
// Shape of the work: the routing is cut into runs of consecutive entries
// with the same expert — with ids sorted by expert, one run per touched
// expert — so the products of a run read the expert's weights once: a wave
// stages each weight row's blocks in LDS and applies them to up to 8 of the
// run's activation rows at a time. The run table (moe_runs.h) is written by
// one extra workgroup of the launch that quantizes the activation
// (launch_act_quantize_moe), so a product is two launches; MXFP4 routings of
// up to 256 entries take one (launch_moe_fp4_fused: the kernel quantizes its
// input rows and finds the runs itself; moe_kq.hip does the same for Q4_K and
// Q6_K).
// The per-unit arithmetic and the reduction are the decode kernel's
// (b32_common.h, wave_sum_dpp), so each pair's result is bit-identical to
// the same product through qmm_forward (times its scale): the reference's
// "matmul_many equals per-job forward" (quantized/mod.rs:743-745).
// MXFP4 rows of up to 128 blocks take moe_fp4_kernel (the matrix-core form);
// the other rows take one of three kernels by row length: moe_b32f_kernel
// (the packed form: an even number of blocks from 64 to 126), moe_b32s_kernel
// (the other rows of up to 4096 values) and moe_b32_kernel (longer rows).
#include "b32_common.h"

namespace qmm {

namespace {

constexpr int kMoeWaves = 4;   // waves per workgroup
constexpr int kMoePairs = 8;   // activation rows a wave applies a staged row to

// runs[0] = number of runs; run r at runs[1 + 3r]: first entry, length, expert
// (written by moe_runs_block, moe_runs.h).

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

// The streaming form: a workgroup of kMoeSWaves waves takes one run and a
// block of the expert's rows, copies the quantized activation rows of up to
// kMoePairs of the run's entries into LDS once, and each wave streams
// kMoeRows consecutive weight rows (their spans of 128 blocks, the next span's
// pieces in flight in registers), applying each to every entry of the chunk.
// The rows a wave streams (rpw) are a launch parameter.
// Per entry the unit arithmetic, the lane's partial across the spans of a
// row and the wave reduction are those of the 1-2 row decode kernel
// (mv_b32s.hip), so each entry's result is bit-identical to qmm_forward of
// its input row, times its scale.
constexpr int kMoeSWaves = 8;  // two workgroups a CU: one streams while the other starts
constexpr int kMoeRing = 2;        // spans in flight per wave
constexpr int kMoeActLoads = 4;    // 16-byte activation pieces a lane copies (k <= 4096; cv0..cv3)
constexpr int kMoeScaleLoads = 2;  // and block scales (cd0, cd1)
static_assert(kMoeSWaves == kMoePairs, "a wave copies each entry's activation row");

template <int FMT>
struct MoeSpan {
  static constexpr int kPieces = (15 + 128 * Fmt32<FMT>::B + 15) / 16;
  static constexpr int kLoads = (kPieces + 63) / 64;
  // a wave's LDS staging buffer: the pieces and the bytes the block reads
  // may touch past the last
  static constexpr int kStage = kPieces * 16 + 16;
  uint4 p[kLoads];
  int off;
  int len;
};

template <int FMT>
__global__ __launch_bounds__(64 * kMoeSWaves) __attribute__((amdgpu_waves_per_eu(4))) void moe_b32s_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int32_t* __restrict__ runs,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m,
    float* __restrict__ dst, int64_t ldd, int rpw) {
  using F = Fmt32<FMT>;
  using Span = MoeSpan<FMT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int k = nb * 32;
  int8_t* const acodes = (int8_t*)smem;                          // [kMoePairs][k]
  float* const ad = (float*)(smem + (size_t)kMoePairs * k);      // [kMoePairs][nb]
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + ((size_t)kMoePairs * (k + nb * 4) + 15) / 16 * 16 + (size_t)wv * Span::kStage;

  const int64_t rb = (int64_t)nb * F::B;
  const int nspan = (nb + 127) / 128;
  const int64_t r0 = ((int64_t)blockIdx.x * kMoeSWaves + wv) * rpw;
  const int64_t nrows = r0 < n ? (n - r0 < rpw ? n - r0 : rpw) : 0;
  const int64_t S = nrows * nspan;
  const Lut32<FMT> lut;
  const uint32_t t0 = lut.t0, t1 = lut.t1, t2 = lut.t2, t3 = lut.t3;
  const int bl = 2 * lane;

  // Runs blockIdx.y, blockIdx.y + gridDim.y, ...: with entries grouped by
  // expert there are at most as many runs as experts and each workgroup
  // takes one; entries in any order are still all computed. The loop and
  // its barriers are uniform over the workgroup.
  const int nruns = __builtin_amdgcn_readfirstlane(runs[0]);
  for (int run = blockIdx.y; run < nruns; run += gridDim.y) {
    // its (first entry, length, expert), one batch of scalar loads
    const int start = __builtin_amdgcn_readfirstlane(runs[1 + 3 * run]);
    const int len = __builtin_amdgcn_readfirstlane(runs[2 + 3 * run]);
    const int e = __builtin_amdgcn_readfirstlane(runs[3 + 3 * run]);
    if (e < 0 || e >= num_experts) continue;
    const uint8_t* We = W + (int64_t)e * estride;

    for (int c0 = 0; c0 < len; c0 += kMoePairs) {
      const int cnt = len - c0 < kMoePairs ? len - c0 : kMoePairs;
      // The wave's weight rows: the loads run kMoeRing spans ahead of the
      // arithmetic; past the wave's last span they read the first bytes of the
      // quantized activation (cached, never used). Every step issues one span's
      // loads and writes all of its pieces, so the compiler counts the loads
      // in flight exactly and waits for the oldest span only. The first spans
      // go out before the entries are looked up.
      int64_t lr = r0;
      int lsp = 0;
      auto load_next = [&](Span& sp) {
        const bool real = lr < r0 + nrows;
        const int b0 = lsp * 128;
        const int blen = real ? (nb - b0 < 128 ? nb - b0 : 128) : 1;
        const uint8_t* pp = real ? We + lr * rb + (int64_t)b0 * F::B : (const uint8_t*)yq;
        sp.off = (int)((uintptr_t)pp & 15);
        sp.len = blen;
        const uint8_t* a0 = pp - sp.off;
        const int pieces = (sp.off + blen * F::B + 15) >> 4;
  #pragma unroll
        for (int c = 0; c < Span::kLoads; c++) {
          const int pc = lane + 64 * c;
          sp.p[c] = ld_stream16(a0 + 16u * (uint32_t)(pc < pieces ? pc : pieces - 1));
        }
        if (++lsp == nspan) {
          lsp = 0;
          lr++;
        }
      };
      Span ring[kMoeRing];
  #pragma unroll
      for (int j = 0; j < kMoeRing; j++) load_next(ring[j]);

      // the chunk's entries: their pair indices (indices clamped into the run),
      // then their routing weights, each one batch
      int pr[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++)
        pr[p] = __builtin_amdgcn_readfirstlane(ids[start + c0 + (p < cnt ? p : cnt - 1)]);
      int64_t out_row[kMoePairs];
      float scale[kMoePairs];
      bool use[kMoePairs];
      int64_t in_row[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) {
        use[p] = p < cnt && pr[p] >= 0 && pr[p] < size_m;
        out_row[p] = use[p] ? pr[p] : 0;
        in_row[p] = use[p] ? (topk_w ? pr[p] : pr[p] / topk) : 0;
      }
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) scale[p] = topk_w ? topk_w[use[p] ? pr[p] : 0] : 1.0f;
      // The chunk's activation rows into LDS (after the previous chunk's
      // reads): entry p is copied by wave p, each lane loading a fixed number
      // of 16-byte code pieces and scales (addresses clamped to the row;
      // k <= 4096, the launcher checks).
      __syncthreads();
      const int cp = wv;  // the entry this wave copies (uniform)
      const int ct = lane;
      const bool cuse = cp < kMoePairs && use[cp < kMoePairs ? cp : 0];
      const int8_t* crow = yq + (cuse ? in_row[cp] * k : 0);
      const float* cdrow = yd + (cuse ? in_row[cp] * nb : 0);
      const int npc = k / 16;
      auto ld_piece = [&](int j) {
        const int i = ct + 64 * j;
        return *(const uint4*)(crow + 16 * (i < npc ? i : npc - 1));
      };
      auto ld_scale = [&](int j) {
        const int i = ct + 64 * j;
        return cdrow[i < nb ? i : nb - 1];
      };
      // named registers (an array here was kept in scratch memory)
      const uint4 cv0 = ld_piece(0), cv1 = ld_piece(1), cv2 = ld_piece(2), cv3 = ld_piece(3);
      const float cd0 = ld_scale(0), cd1 = ld_scale(1);
      if (cuse) {
        auto st_piece = [&](int j, const uint4& v) {
          const int i = ct + 64 * j;
          if (i < npc) *(uint4*)(acodes + cp * k + 16 * i) = v;
        };
        auto st_scale = [&](int j, float v) {
          const int i = ct + 64 * j;
          if (i < nb) ad[cp * nb + i] = v;
        };
        st_piece(0, cv0);
        st_piece(1, cv1);
        st_piece(2, cv2);
        st_piece(3, cv3);
        st_scale(0, cd0);
        st_scale(1, cd1);
      }
      __syncthreads();
      int64_t R = r0;
      int sp = 0;
      float acc[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) acc[p] = 0.0f;
      // Staging and the next span's load issue run at a raised wave priority,
      // the unit arithmetic at the default: a wave's requests go out ahead of
      // the other waves' vector work (C4's grouped launches 1-2% faster).
      auto step = [&](Span& cur, int64_t sigma) {
        __builtin_amdgcn_s_setprio(1);
        wave_lds_sync();
  #pragma unroll
        for (int c = 0; c < Span::kLoads; c++) {
          const int pc = lane + 64 * c;
          *(uint4*)(buf + 16 * (pc < Span::kPieces ? pc : Span::kPieces - 1)) = cur.p[c];
        }
        wave_lds_sync();
        const int off = cur.off, blen = cur.len;
        load_next(cur);
        __builtin_amdgcn_s_setprio(0);
        if (sigma >= S) return;
        if (bl < blen) {
          const bool two = bl + 1 < blen;
          uint32_t q0[8], q1[8];
          float dx0, dx1;
          F::decode(buf, off + bl * F::B, q0, dx0, t0, t1, t2, t3);
          if (two) {
            F::decode(buf, off + (bl + 1) * F::B, q1, dx1, t0, t1, t2, t3);
          } else {
  #pragma unroll
            for (int t = 0; t < 8; t++) q1[t] = 0;
            dx1 = 0.0f;
          }
          const int gb = sp * 128 + bl;
  #pragma unroll
          for (int p = 0; p < kMoePairs; p++) {
            if (!use[p]) continue;
            Act64 a;
            const int4* yp = (const int4*)(acodes + p * k + gb * 32);
            const int4 a0 = yp[0], a1 = yp[1];
            a.y[0][0] = a0.x; a.y[0][1] = a0.y; a.y[0][2] = a0.z; a.y[0][3] = a0.w;
            a.y[0][4] = a1.x; a.y[0][5] = a1.y; a.y[0][6] = a1.z; a.y[0][7] = a1.w;
            a.dy[0] = ad[p * nb + gb];
            if (two) {
              const int4 b0 = yp[2], b1 = yp[3];
              a.y[1][0] = b0.x; a.y[1][1] = b0.y; a.y[1][2] = b0.z; a.y[1][3] = b0.w;
              a.y[1][4] = b1.x; a.y[1][5] = b1.y; a.y[1][6] = b1.z; a.y[1][7] = b1.w;
              a.dy[1] = ad[p * nb + gb + 1];
            } else {
  #pragma unroll
              for (int t = 0; t < 8; t++) a.y[1][t] = 0;
              a.dy[1] = 0.0f;
            }
            acc[p] = b32_unit(q0, q1, dx0, dx1, a, acc[p]);
          }
        }
        if (++sp == nspan) {
  #pragma unroll
          for (int p = 0; p < kMoePairs; p++) {
            if (!use[p]) continue;
            const float v = wave_sum_dpp(acc[p]);
            if (lane == 0) dst[out_row[p] * ldd + R] = __fmul_rn(v, scale[p]);
            acc[p] = 0.0f;
          }
          sp = 0;
          R++;
        }
      };
      for (int64_t sigma = 0; sigma < S; sigma += kMoeRing) {
  #pragma unroll
        for (int j = 0; j < kMoeRing; j++) step(ring[j], sigma + j);
      }
    }
  }
}

// The packed form, for rows of an even number of blocks from 64 to 126
// (C4's 2880-value rows are 90 blocks: 45 units of two, so the streaming form
// leaves 19 of 64 lanes without a unit). A wave's rows are contiguous bytes
// and, with an even block count, a sequence of equal two-block units: step j
// gives lane L unit 64 j + L of that sequence, in whichever row it falls, so
// every lane holds one. A unit's value, b32_unit(..., 0), is the partial that
// lane (unit mod units-a-row) holds in the streaming form (such a row is one
// span, so that lane's partial is its one unit, and the lanes past the row's
// units hold 0). When a row's last unit has been computed, lane v of the wave
// fetches the value of the row's unit v (ds_bpermute, from this step's lanes
// or the previous step's) and the wave sums them with wave_sum_dpp: the same
// 64 partials in the same lanes, so each entry's result has the streaming
// form's bits, and the decode kernel's.
constexpr int kMoeRec = 80;  // LDS bytes of one activation unit in the packed form

template <int FMT>
__global__ __launch_bounds__(64 * kMoeSWaves) __attribute__((amdgpu_waves_per_eu(4))) void moe_b32f_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int32_t* __restrict__ runs,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m,
    float* __restrict__ dst, int64_t ldd, int rpw) {
  using F = Fmt32<FMT>;
  using Span = MoeSpan<FMT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int k = nb * 32;
  const int upr = nb >> 1;      // units a row, 32..63
  constexpr int kUB = 2 * F::B;  // bytes a unit
  // the chunk's activation rows: per entry and unit one 80-byte record, the
  // unit's 64 codes then its two block scales (80 bytes apart, the 16 lanes
  // of one LDS read phase fall on distinct banks; 64 apart they met 4 ways)
  uint8_t* const arec = smem;  // [kMoePairs][upr][80]
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + (size_t)kMoePairs * upr * kMoeRec + (size_t)wv * Span::kStage;

  const int64_t rb = (int64_t)nb * F::B;
  const int64_t r0 = ((int64_t)blockIdx.x * kMoeSWaves + wv) * rpw;
  const int nrows = r0 < n ? (int)(n - r0 < rpw ? n - r0 : rpw) : 0;
  const int U = nrows * upr;  // the wave's units
  const int nsteps = (U + 63) >> 6;
  const Lut32<FMT> lut;
  const uint32_t t0 = lut.t0, t1 = lut.t1, t2 = lut.t2, t3 = lut.t3;

  const int nruns = __builtin_amdgcn_readfirstlane(runs[0]);
  for (int run = blockIdx.y; run < nruns; run += gridDim.y) {
    const int start = __builtin_amdgcn_readfirstlane(runs[1 + 3 * run]);
    const int len = __builtin_amdgcn_readfirstlane(runs[2 + 3 * run]);
    const int e = __builtin_amdgcn_readfirstlane(runs[3 + 3 * run]);
    if (e < 0 || e >= num_experts) continue;
    const uint8_t* Wr = W + (int64_t)e * estride + r0 * rb;  // the wave's first row

    for (int c0 = 0; c0 < len; c0 += kMoePairs) {
      const int cnt = len - c0 < kMoePairs ? len - c0 : kMoePairs;
      // Step ls's bytes: units 64 ls .. of the wave's sequence; past the last
      // step the loads read the first bytes of the quantized activation
      // (cached, never used), so every step issues the same loads.
      int ls = 0;
      auto load_next = [&](Span& sp) {
        const int u0 = 64 * ls;
        const bool real = u0 < U;
        const int units = real ? (U - u0 < 64 ? U - u0 : 64) : 1;
        const uint8_t* pp = real ? Wr + (int64_t)u0 * kUB : (const uint8_t*)yq;
        sp.off = (int)((uintptr_t)pp & 15);
        sp.len = units;
        const uint8_t* a0 = pp - sp.off;
        const int pieces = (sp.off + units * kUB + 15) >> 4;
  #pragma unroll
        for (int c = 0; c < Span::kLoads; c++) {
          const int pc = lane + 64 * c;
          sp.p[c] = ld_stream16(a0 + 16u * (uint32_t)(pc < pieces ? pc : pieces - 1));
        }
        ls++;
      };
      Span ring[kMoeRing];
  #pragma unroll
      for (int j = 0; j < kMoeRing; j++) load_next(ring[j]);

      int pr[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++)
        pr[p] = __builtin_amdgcn_readfirstlane(ids[start + c0 + (p < cnt ? p : cnt - 1)]);
      int64_t out_row[kMoePairs];
      float scale[kMoePairs];
      bool use[kMoePairs];
      int64_t in_row[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) {
        use[p] = p < cnt && pr[p] >= 0 && pr[p] < size_m;
        out_row[p] = use[p] ? pr[p] : 0;
        in_row[p] = use[p] ? (topk_w ? pr[p] : pr[p] / topk) : 0;
      }
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) scale[p] = topk_w ? topk_w[use[p] ? pr[p] : 0] : 1.0f;
      // the chunk's activation rows into LDS, as the streaming form copies them
      __syncthreads();
      const int cp = wv;
      const bool cuse = use[cp];
      const int8_t* crow = yq + (cuse ? in_row[cp] * k : 0);
      const float* cdrow = yd + (cuse ? in_row[cp] * nb : 0);
      const int npc = k / 16;
      auto ld_piece = [&](int j) {
        const int i = lane + 64 * j;
        return *(const uint4*)(crow + 16 * (i < npc ? i : npc - 1));
      };
      auto ld_scale = [&](int j) {
        const int i = lane + 64 * j;
        return cdrow[i < nb ? i : nb - 1];
      };
      const uint4 cv0 = ld_piece(0), cv1 = ld_piece(1), cv2 = ld_piece(2), cv3 = ld_piece(3);
      const float cd0 = ld_scale(0), cd1 = ld_scale(1);
      if (cuse) {
        uint8_t* const mine = arec + (size_t)cp * upr * kMoeRec;
        auto st_piece = [&](int j, const uint4& v) {
          const int i = lane + 64 * j;  // piece i & 3 of unit i >> 2
          if (i < npc) *(uint4*)(mine + kMoeRec * (i >> 2) + 16 * (i & 3)) = v;
        };
        auto st_scale = [&](int j, float v) {
          const int i = lane + 64 * j;  // block i: scale i & 1 of unit i >> 1
          if (i < nb) *(float*)(mine + kMoeRec * (i >> 1) + 64 + 4 * (i & 1)) = v;
        };
        st_piece(0, cv0);
        st_piece(1, cv1);
        st_piece(2, cv2);
        st_piece(3, cv3);
        st_scale(0, cd0);
        st_scale(1, cd1);
      }
      __syncthreads();

      // lane L's unit within its row (64 j + L mod upr, kept step to step)
      int vl = lane < upr ? lane : lane - upr;
      int rr = 0;  // the first row not yet summed
      float prev[kMoePairs];
  #pragma unroll
      for (int p = 0; p < kMoePairs; p++) prev[p] = 0.0f;
      auto step = [&](Span& cur, int j) {
        __builtin_amdgcn_s_setprio(1);
        wave_lds_sync();
  #pragma unroll
        for (int c = 0; c < Span::kLoads; c++) {
          const int pc = lane + 64 * c;
          *(uint4*)(buf + 16 * (pc < Span::kPieces ? pc : Span::kPieces - 1)) = cur.p[c];
        }
        wave_lds_sync();
        const int off = cur.off, units = cur.len;
        load_next(cur);
        __builtin_amdgcn_s_setprio(0);
        if (j >= nsteps) return;
        float val[kMoePairs];
  #pragma unroll
        for (int p = 0; p < kMoePairs; p++) val[p] = 0.0f;
        if (lane < units) {
          uint32_t q0[8], q1[8];
          float dx0, dx1;
          F::decode(buf, off + lane * kUB, q0, dx0, t0, t1, t2, t3);
          F::decode(buf, off + lane * kUB + F::B, q1, dx1, t0, t1, t2, t3);
  #pragma unroll
          for (int p = 0; p < kMoePairs; p++) {
            if (p >= cnt) break;  // the chunk's entries come first
            if (!use[p]) continue;
            Act64 a;
            const uint8_t* rec = arec + ((size_t)p * upr + vl) * kMoeRec;
            const int4* yp = (const int4*)rec;
            const int4 a0 = yp[0], a1 = yp[1], b0 = yp[2], b1 = yp[3];
            const float2 dd = *(const float2*)(rec + 64);
            a.y[0][0] = a0.x; a.y[0][1] = a0.y; a.y[0][2] = a0.z; a.y[0][3] = a0.w;
            a.y[0][4] = a1.x; a.y[0][5] = a1.y; a.y[0][6] = a1.z; a.y[0][7] = a1.w;
            a.y[1][0] = b0.x; a.y[1][1] = b0.y; a.y[1][2] = b0.z; a.y[1][3] = b0.w;
            a.y[1][4] = b1.x; a.y[1][5] = b1.y; a.y[1][6] = b1.z; a.y[1][7] = b1.w;
            a.dy[0] = dd.x;
            a.dy[1] = dd.y;
            val[p] = b32_unit(q0, q1, dx0, dx1, a, 0.0f);
          }
        }
        // the rows whose last unit is in this step (at most two: upr >= 32);
        // row r's unit v sits in lane r upr - 64 j + v of this step, or, where
        // that is negative, 64 lanes on in the previous step
        const int u0 = 64 * j;
        for (; rr < nrows && (rr + 1) * upr <= u0 + 64; rr++) {
          const int base = rr * upr - u0;  // > -64
          const int s = base + lane;
          const bool mine = lane < upr;
  #pragma unroll
          for (int p = 0; p < kMoePairs; p++) {
            if (p >= cnt) break;  // the chunk's entries come first
            if (!use[p]) continue;
            const float fc = __int_as_float(__builtin_amdgcn_ds_bpermute((s & 63) << 2, __float_as_int(val[p])));
            float v = fc;
            if (base < 0) {
              const float fp = __int_as_float(__builtin_amdgcn_ds_bpermute(((s + 64) & 63) << 2, __float_as_int(prev[p])));
              v = s < 0 ? fp : fc;
            }
            v = wave_sum_dpp(mine ? v : 0.0f);
            if (lane == 0) dst[out_row[p] * ldd + r0 + rr] = __fmul_rn(v, scale[p]);
          }
        }
  #pragma unroll
        for (int p = 0; p < kMoePairs; p++) prev[p] = val[p];
        vl += 64 - upr;
        if (vl >= upr) vl -= upr;
      };
      for (int j = 0; j < nsteps; j += kMoeRing) {
  #pragma unroll
        for (int jj = 0; jj < kMoeRing; jj++) step(ring[jj], j + jj);
      }
    }
  }
}

// The matrix-core form, for MXFP4 rows of up to 128 blocks. The weight's
// nibbles are E2M1 codes, so a block's integer dot with the Q8_0 codes is a
// product on the matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4: B the
// weight bytes as they lie in the block, A E4M3, both scales 2^0) once each
// activation code y = 16 h + l (h in [-8, 7], l in [0, 15]) is given as two
// exact E4M3 codes:
//     sum_i t(w_i) y_i = 2 (16 H + L),  H = sum_i e2m1(w_i) h_i,  L = sum_i e2m1(w_i) l_i
// (t = kMxfp4Values = 2 e2m1). Every product and partial sum is a multiple
// of 1/2 below 2^12, so the matrix-core sums are exact and s_b = 2 (16 H + L)
// is the decode kernel's integer sum. The product's 16 columns are 16 weight
// rows and its 128 K values 4 blocks; its 16 rows are 4 entries x 4 block
// slots, row (p, s) holding entry p's codes in slot s's 32 K values and zeros
// in the other 96, so output (p, s; j) is block s's sum alone. The weight
// block's byte i holds values i (low nibble) and i + 16 (high), and the
// matrix cores read byte i as K 2i, 2i+1, so the activation codes are laid
// out in that order. Output lane (p, j) forms each block's
// p_b = (dx_b dy_b) s_b and each unit's 0 + (p_2u + p_2u+1) as b32_unit
// does, and sums the row's units in wave_sum_dpp's tree (pairs, pairs of
// pairs, ..., over 64 leaves, +0 past the row's units), so each entry's
// result has the decode kernel's bits.
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kMoeFusedMaxEntries = 256;  // routings the fused form takes (each wave scans them)
constexpr int kFp4Pairs = 4;       // entries a pass: the product's 4 row groups
constexpr int kFp4Rows = 16;       // weight rows a wave: the product's 16 columns
// A step takes 16 blocks (272 bytes) of each of the wave's rows: the
// 16-byte pieces from the one holding its first byte to the one holding its
// last, row r's at piece 19 r .. of the wave's stage buffer.
constexpr int kFp4StepBlocks = 16;
constexpr int kFp4StepBytes = 17 * kFp4StepBlocks;
constexpr int kFp4SegPieces = (15 + kFp4StepBytes + 15) / 16;  // 272 bytes at any alignment: 18
constexpr int kFp4Slots = kFp4Rows * kFp4SegPieces;  // pieces a step: 288
constexpr int kFp4Loads = (kFp4Slots + 63) / 64;     // a lane's: 5
// a row's 18 pieces 304 bytes apart (12 banks on: the 16 rows of a read on
// distinct banks; a stride of 10 pieces to 8 blocks put rows 8 apart, whose
// bytes also share their alignment, on the same ones)
constexpr int kFp4RowStride = 19;
constexpr int kFp4Stage = kFp4Rows * kFp4RowStride * 16 + 16;  // and the dword past the last that lds_words reads
constexpr int kFp4Rec = 64;  // LDS bytes of an entry's block: h0 h1 l0 l1, 16 bytes each
constexpr int kFp4Ring = 2;  // steps in flight per wave
// LDS: 64 zero bytes, then entry p's records at kFp4Codes + p P (P = 64 nb
// rounded up to 64 mod 256): in each 16-lane phase of an A read the four
// lanes that read codes fall on distinct banks, and the others read zeros
// (at 32 for the h codes, at 0 for the l codes) on banks of their own
constexpr int kFp4Codes = 64;
__host__ __device__ inline int fp4_entry_stride(int nb) { return 64 * nb + (64 - 64 * (nb % 4) + 256) % 256; }
// the scales' rows: whole steps, the blocks past the row zero
__host__ __device__ inline int fp4_dy_stride(int nb) { return (nb + kFp4StepBlocks - 1) / kFp4StepBlocks * kFp4StepBlocks; }

struct Fp4Span {
  uint4 p[kFp4Loads];
};

inline size_t moe_fp4_lds(int64_t nb) {
  return kFp4Codes + (size_t)kFp4Pairs * fp4_entry_stride((int)nb) + 16 * (size_t)fp4_dy_stride((int)nb) +
         (size_t)kMoeSWaves * kFp4Stage;
}

// kFused: the kernel takes the f32 input rows and the routing's expert ids
// itself (the one launch of a small routing): each wave finds its runs in
// expert_ids, and the chunk's codes and scales are quantized in the set-up
// with the quantizer's own arithmetic (q8_0_kernel, quantize.hip), so they
// have its bits. Otherwise the quantized planes (yq, yd) and the run table
// come from launch_act_quantize_moe.
template <bool kFused>
__global__ __launch_bounds__(64 * kMoeSWaves) __attribute__((amdgpu_waves_per_eu(4))) void moe_fp4_kernel(
    const uint8_t* __restrict__ W, int64_t n, int nb, int64_t estride, int num_experts,
    const int8_t* __restrict__ yq, const float* __restrict__ yd, const int32_t* __restrict__ runs,
    const float* __restrict__ xa, int64_t x_stride, const int32_t* __restrict__ expert_ids, int xvec,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m,
    float* __restrict__ dst, int64_t ldd) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // LDS: zeros; the chunk's codes, record (p, b) at kFp4Codes + p P + 64 b;
  // the block scales dy[p][b] (rows of dys floats); the waves' stage buffers
  const int k = nb * 32;
  const int dys = fp4_dy_stride(nb);
  const int P = fp4_entry_stride(nb);
  float* const dyt = (float*)(smem + kFp4Codes + kFp4Pairs * P);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = (uint8_t*)(dyt + kFp4Pairs * dys) + wv * kFp4Stage;
  const int64_t rb = (int64_t)nb * 17;
  const int64_t r0 = ((int64_t)blockIdx.x * kMoeSWaves + wv) * kFp4Rows;
  const int nrows = r0 < n ? (int)(n - r0 < kFp4Rows ? n - r0 : kFp4Rows) : 0;
  const int nsteps = (nb + kFp4StepBlocks - 1) / kFp4StepBlocks;

  // the zeros, and the scales past the row (blocks past the row then give
  // (dx * 0) * s = +-0)
  for (int i = threadIdx.x; i < kFp4Codes / 16 + kFp4Pairs * dys / 4; i += blockDim.x)
    *(uint4*)(i < kFp4Codes / 16 ? smem + 16 * i : (uint8_t*)dyt + 16 * (i - kFp4Codes / 16)) = make_uint4(0u, 0u, 0u, 0u);
  // E4M3 codes of l = nibble and of h = nibble - 16 (nibble >= 8), for lut16_at
  const uint32_t cl0 = 0x44403800u, cl1 = 0x4E4C4A48u, cl2 = 0x53525150u, cl3 = 0x57565554u;
  const uint32_t ch2 = 0xCACCCED0u, ch3 = 0xB8C0C4C8u;

  const int jn = lane & 15;    // the lane's weight row: its B column and output column
  const int gk = lane >> 4;    // B: the block slot of the lane's 16 bytes; A: its K group
  const int pa = jn >> 2, sa = lane & 3;  // A: the entry and block slot of the lane's row
  // A's K group gk holds K [16 gk, +16) in bytes 0-15 (block slot gk / 2) and
  // K [64 + 16 gk, +16) in bytes 16-31 (slot 2 + gk / 2): the lane's row has
  // codes in one of them exactly when (sa & 1) == gk / 2, the low half for
  // slots 0 and 1; the other half is zeros
  const bool aslot = (sa & 1) == (gk >> 1);
  const bool alow = sa < 2;
  const int aoff = 16 * (gk & 1);
  const int po = gk;  // output: the lane's entry
  const int rowc = jn < nrows ? jn : nrows - 1;
  // load c of a step: piece lpc of the row at byte lro from the wave's
  // first (packed: lro in bits 0-15, as the wave's rows span < 32 KiB, lpc
  // 16-19)
  uint32_t lpk[kFp4Loads];
#pragma unroll
  for (int c = 0; c < kFp4Loads; c++) {
    const int s = lane + 64 * c < kFp4Slots ? lane + 64 * c : kFp4Slots - 1;
    const int r = s / kFp4SegPieces;
    lpk[c] = (uint32_t)((r < nrows ? r : nrows - 1) * (int)rb) | (uint32_t)(s - r * kFp4SegPieces) << 16;
  }

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
    const uint8_t* Wr = W + (int64_t)e * estride + r0 * rb;  // the wave's first row

    for (int c0 = 0; c0 < len; c0 += kFp4Pairs) {
      const int cnt = len - c0 < kFp4Pairs ? len - c0 : kFp4Pairs;
      int pr[kFp4Pairs];
      bool use[kFp4Pairs];
      int64_t in_row[kFp4Pairs];
#pragma unroll
      for (int p = 0; p < kFp4Pairs; p++) {
        pr[p] = __builtin_amdgcn_readfirstlane(ids[start + c0 + (p < cnt ? p : cnt - 1)]);
        use[p] = p < cnt && pr[p] >= 0 && pr[p] < size_m;
        in_row[p] = use[p] ? (topk_w ? pr[p] : pr[p] / topk) : 0;
      }
      // step ls's loads; past the last step they read the wave's first bytes
      // again (cached, never used). The first steps' loads
      // are issued before the chunk's codes are laid out. (32-bit offsets
      // from the 16-byte aligned address at or below the uniform base, so
      // none is negative; a piece past the step's last is replaced by its
      // last, so no load touches bytes of another step.)
      int ls = 0;
      auto load_next = [&](Fp4Span& sp) {
        const bool real = ls < nsteps;
        const uint8_t* base = Wr;
        const uint32_t bofs = (uint32_t)(uintptr_t)base & 15u;
        const uint8_t* const ba = base - bofs;
        const int blen = real ? (nb - kFp4StepBlocks * ls < kFp4StepBlocks ? nb - kFp4StepBlocks * ls : kFp4StepBlocks) : 1;
        const uint32_t st = bofs + (real ? (uint32_t)kFp4StepBytes * (uint32_t)ls : 0u);
#pragma unroll
        for (int c = 0; c < kFp4Loads; c++) {
          const uint32_t rel = (real ? lpk[c] & 0xFFFFu : 0u) + st;  // the step's first byte, from ba
          const uint32_t pieces = ((rel & 15u) + 17u * (uint32_t)blen + 15u) >> 4;
          const uint32_t pc = lpk[c] >> 16;
          sp.p[c] = ld_stream16(ba + ((rel & ~15u) + 16u * (pc < pieces ? pc : pieces - 1u)));
        }
        ls++;
      };
      Fp4Span ring[kFp4Ring];
      if (nrows > 0) {
#pragma unroll
        for (int j = 0; j < kFp4Ring; j++) load_next(ring[j]);
      }

      // the chunk's codes into LDS, as E4M3 h and l codes in the weight's K order
      __syncthreads();
      for (int t = threadIdx.x; t < kFp4Pairs * nb * 2; t += blockDim.x) {
        const int p = t / (2 * nb), b = (t - p * 2 * nb) >> 1, q = t & 1;
        bool u = false;
        int64_t ir = 0;
#pragma unroll
        for (int pp = 0; pp < kFp4Pairs; pp++)
          if (p == pp) u = use[pp], ir = in_row[pp];
        if (!u) continue;
        uint2 lo, hi;  // the codes of values 8q .., 16 + 8q ..
        if (kFused) {
          // q8_0_kernel's block: the maximum over 4-value groups as bits,
          // across the pair of lanes of this block (both run this task)
          const float* xr = xa + ir * x_stride + 32 * b + 8 * q;
          float v[16];
          if (xvec) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
              const float4 f = *(const float4*)(xr + (g < 2 ? 4 * g : 8 + 4 * g));
              v[4 * g] = f.x, v[4 * g + 1] = f.y, v[4 * g + 2] = f.z, v[4 * g + 3] = f.w;
            }
          } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = xr[i < 8 ? i : 8 + i];
          }
          uint32_t ab = 0u;
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const float a = fmaxf(fmaxf(fabsf(v[4 * g]), fabsf(v[4 * g + 1])), fmaxf(fabsf(v[4 * g + 2]), fabsf(v[4 * g + 3])));
            ab = max(ab, __float_as_uint(fmaxf(a, 0.0f)));
          }
          ab = max(ab, (uint32_t)__shfl_xor((int)ab, 1, 64));
          const float d = __uint_as_float(ab) / 127.0f;
          const float id = d != 0.0f ? 1.0f / d : 0.0f;
          uint32_t cw[4];
#pragma unroll
          for (int g = 0; g < 4; g++)
            cw[g] = pack4_i8(q8_0_code(v[4 * g] * id), q8_0_code(v[4 * g + 1] * id), q8_0_code(v[4 * g + 2] * id),
                             q8_0_code(v[4 * g + 3] * id));
          lo = make_uint2(cw[0], cw[1]);
          hi = make_uint2(cw[2], cw[3]);
          if (q == 0) dyt[p * dys + b] = h2f(f2h(d));  // Q8_0's block scale is an f16
        } else {
          const int8_t* src = yq + ir * k + 32 * b + 8 * q;
          lo = *(const uint2*)src;
          hi = *(const uint2*)(src + 16);
        }
        uint32_t x[4];  // K 16q + 2i: value 8q + i; K 16q + 2i + 1: value 16 + 8q + i
        x[0] = __builtin_amdgcn_perm(hi.x, lo.x, 0x05010400u);
        x[1] = __builtin_amdgcn_perm(hi.x, lo.x, 0x07030602u);
        x[2] = __builtin_amdgcn_perm(hi.y, lo.y, 0x05010400u);
        x[3] = __builtin_amdgcn_perm(hi.y, lo.y, 0x07030602u);
        uint32_t h[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          h[i] = (uint32_t)lut16_at(x[i], 4, cl0, cl1, ch2, ch3);
          l[i] = (uint32_t)lut16_at(x[i], 0, cl0, cl1, cl2, cl3);
        }
        uint8_t* rec = smem + kFp4Codes + P * p + kFp4Rec * b;
        *(uint4*)(rec + 16 * q) = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4*)(rec + 32 + 16 * q) = make_uint4(l[0], l[1], l[2], l[3]);
      }
      for (int t = threadIdx.x; !kFused && t < kFp4Pairs * nb; t += blockDim.x) {
        const int p = t / nb, b = t - p * nb;
        bool u = false;
        int64_t ir = 0;
#pragma unroll
        for (int pp = 0; pp < kFp4Pairs; pp++)
          if (p == pp) u = use[pp], ir = in_row[pp];
        if (u) dyt[p * dys + b] = yd[ir * nb + b];
      }
      __syncthreads();
      if (nrows == 0) continue;

      bool a_on = false;
#pragma unroll
      for (int p = 0; p < kFp4Pairs; p++)
        if (pa == p) a_on = aslot && use[p];
      const uint32_t browlo = (uint32_t)(uintptr_t)Wr + (uint32_t)(rowc * (int)rb);  // row rowc's address, low bits

      // wave_sum_dpp's tree over the row's 64 leaves (lane L's leaf is unit
      // L): group t's node holds 2 leaves, step j's four groups give its node
      // of 8, x = (g0 + g1) + (g2 + g3), and push(x, j) folds it in as a
      // binary counter over j: v8 .. v32 keep the pending nodes of 8 .. 32
      // leaves (every sum formed, the stores selected: j is uniform)
      float v8 = 0.0f, v16 = 0.0f, v32 = 0.0f, res = 0.0f;
      auto push = [&](float x, int j) {
        const bool b0 = j & 1, b1 = (j & 3) == 3, b2 = (j & 7) == 7;
        const float x16 = v8 + x, x32 = v16 + x16, x64 = v32 + x32;
        v8 = b0 ? v8 : x;
        v16 = b0 && !(j & 2) ? x16 : v16;
        v32 = b1 && !(j & 4) ? x32 : v32;
        res = b2 ? x64 : res;
      };
      auto step = [&](Fp4Span& cur, int j) {
        __builtin_amdgcn_sched_barrier(0);
        wave_lds_sync();
#pragma unroll
        for (int c = 0; c < kFp4Loads; c++)
          if (lane + 64 * c < kFp4Slots)
            *(uint4*)(buf + 16 * (lane + 64 * c + (kFp4RowStride - kFp4SegPieces) * ((lane + 64 * c) / kFp4SegPieces))) = cur.p[c];
        wave_lds_sync();
        load_next(cur);
        if (j >= nsteps) return;
        const int b0 = kFp4StepBlocks * j;
        const int off = (int)((browlo + 17u * (uint32_t)b0) & 15u);
        const int rbase = 16 * kFp4RowStride * jn + off;  // row jn's block b0 in the stage buffer
        float g[kFp4StepBlocks / 4];
#pragma unroll
        for (int t = 0; t < kFp4StepBlocks / 4; t++) {
          // group t: blocks bg .. bg + 3 (past the row: zero codes, zero scales)
          const int bg = b0 + 4 * t;
          uint32_t bw[4];
          lds_words<4>(buf, rbase + 17 * (4 * t + gk) + 1, bw);
          const v4i_t b4 = {(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]};
          const v8i_t bv = __builtin_shufflevector(b4, b4, 0, 1, 2, 3, -1, -1, -1, -1);  // E2M1: 4 registers read
          const int ab = bg + sa;
          const bool on = a_on && ab < nb;
          const int ao = kFp4Codes + P * pa + kFp4Rec * ab + aoff;  // the h codes; the l codes 32 on
          const bool lo_on = on && alow, hi_on = on && !alow;
          // s_b = 32 H + 2 L = sum_i t(w_i) y_i, exact: the A scales 2^5 and 2^1
          const v4f_t z = {0.0f, 0.0f, 0.0f, 0.0f};
          const v4i_t h0 = *(const v4i_t*)(smem + (lo_on ? ao : 32)), h1 = *(const v4i_t*)(smem + (hi_on ? ao : 32));
          const v8i_t ah = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
          v4f_t sb = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ah, bv, z, 0, 4, 0, 132, 0, 127);
          __builtin_amdgcn_sched_barrier(0);  // one A operand live at a time
          const v4i_t l0 = *(const v4i_t*)(smem + (lo_on ? ao + 32 : 0)), l1 = *(const v4i_t*)(smem + (hi_on ? ao + 32 : 0));
          const v8i_t al = __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
          sb = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(al, bv, sb, 0, 4, 0, 128, 0, 127);
          const float4 dy = *(const float4*)(dyt + po * dys + bg);
          const float dyv[4] = {dy.x, dy.y, dy.z, dy.w};
          float pb[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            // e8m0_half: 2^(e - 128), exact (subnormal for e < 2)
            const float dx = __builtin_amdgcn_ldexpf(1.0f, (int)buf[rbase + 17 * (4 * t + i)] - 128);
            pb[i] = (dx * dyv[i]) * sb[i];
          }
          // = (0 + (p0 + p1)) + (0 + (p2 + p3)) bit for bit: a p here differs
          // from the decode kernel's only in the sign of a zero
          g[t] = 0.0f + ((pb[0] + pb[1]) + (pb[2] + pb[3]));
          __builtin_amdgcn_sched_barrier(0);  // one group's operands live at a time
        }
        push((g[0] + g[1]) + (g[2] + g[3]), j);
      };
      for (int j = 0; j < nsteps; j += kFp4Ring) {
#pragma unroll
        for (int jj = 0; jj < kFp4Ring; jj++) step(ring[jj], j + jj);
      }
      for (int j = nsteps; j < 64 / (kFp4StepBlocks / 2); j++) push(0.0f + 0.0f, j);
      bool o_use = false;
      int64_t o_row = 0;
#pragma unroll
      for (int p = 0; p < kFp4Pairs; p++)
        if (po == p) o_use = use[p], o_row = use[p] ? pr[p] : 0;
      if (o_use && jn < nrows) dst[o_row * ldd + r0 + jn] = __fmul_rn(res, topk_w ? topk_w[o_row] : 1.0f);
    }
  }
}

hipError_t launch_moe_fp4(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                          const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                          float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int nb = (int)(k / 32);
  const int64_t estride = n * nb * 17;
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  const int64_t rows_per_wg = (int64_t)kMoeSWaves * kFp4Rows;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = moe_fp4_lds(nb);
  constexpr auto* kfn = &moe_fp4_kernel<false>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kMoeSWaves, lds, st>>>((const uint8_t*)w, n, nb, estride, num_experts, p.codes, p.d, runs,
                                          nullptr, 0, nullptr, 0, ids, topk_w, topk, (int)size_m, dst, ldd);
  return hipGetLastError();
}

// Rows the matrix-core form takes: up to 128 blocks (the tree's 64 leaves).
inline bool moe_fp4_takes(int64_t k) { return k / 32 <= 128 && moe_fp4_lds(k / 32) <= 160 * 1024; }

}  // namespace

bool moe_fp4_fused_takes(int type, int64_t k, int64_t size_m) {
  return type == T_MXFP4 && moe_fp4_takes(k) && size_m <= kMoeFusedMaxEntries;
}

hipError_t launch_moe_fp4_fused(const void* w, int num_experts, int64_t n, int64_t k, const float* x,
                                int64_t x_stride, const int32_t* expert_ids, const int32_t* ids, const float* topk_w,
                                int topk, int64_t size_m, float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int nb = (int)(k / 32);
  const int64_t estride = n * nb * 17;
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  const int64_t rows_per_wg = (int64_t)kMoeSWaves * kFp4Rows;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = moe_fp4_lds(nb);
  const int xvec = ((uintptr_t)x % 16 == 0) && (x_stride % 4 == 0);
  constexpr auto* kfn = &moe_fp4_kernel<true>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kMoeSWaves, lds, st>>>((const uint8_t*)w, n, nb, estride, num_experts, nullptr, nullptr, nullptr,
                                          x, x_stride, expert_ids, xvec, ids, topk_w, topk, (int)size_m, dst, ldd);
  return hipGetLastError();
}

namespace {

template <int FMT>
hipError_t launch_moe_s(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                        const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                        float* dst, int64_t ldd, int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int nb = (int)(k / 32);
  const int64_t estride = n * nb * Fmt32<FMT>::B;
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  // rows a wave: 8 (measured against 12-23 at C4's shapes: longer rows per
  // wave lengthen each wave's chain of two-rows-in-flight steps more than
  // fewer workgroups save in fills)
  (void)cus;
  const int64_t rpw = 8;
  const int64_t rows_per_wg = (int64_t)kMoeSWaves * rpw;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = ((size_t)kMoePairs * (k + nb * 4) + 15) / 16 * 16 + (size_t)kMoeSWaves * MoeSpan<FMT>::kStage;
  constexpr auto* kfn = &moe_b32s_kernel<FMT>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kMoeSWaves, lds, st>>>((const uint8_t*)w, n, nb, estride, num_experts, p.codes, p.d, runs, ids,
                                          topk_w, topk, (int)size_m, dst, ldd, (int)rpw);
  return hipGetLastError();
}

template <int FMT>
hipError_t launch_moe_f(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                        const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                        float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int nb = (int)(k / 32);
  const int64_t estride = n * nb * Fmt32<FMT>::B;
  const int64_t gy = size_m < num_experts ? size_m : num_experts;
  // rows a wave: 16 (C4: 720 units, 12 steps of 64, no step partly empty
  // but the last; 8 rows measured 1% slower, 10 and 12 rows, whose last
  // steps hold few units, 10-15% slower)
  const int64_t rpw = 16;
  const int64_t rows_per_wg = (int64_t)kMoeSWaves * rpw;
  const dim3 grid((unsigned)((n + rows_per_wg - 1) / rows_per_wg), (unsigned)(gy < 1 ? 1 : gy));
  const size_t lds = (size_t)kMoePairs * (nb / 2) * kMoeRec + (size_t)kMoeSWaves * MoeSpan<FMT>::kStage;
  constexpr auto* kfn = &moe_b32f_kernel<FMT>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kMoeSWaves, lds, st>>>((const uint8_t*)w, n, nb, estride, num_experts, p.codes, p.d, runs, ids,
                                          topk_w, topk, (int)size_m, dst, ldd, (int)rpw);
  return hipGetLastError();
}

// Rows the packed form takes: an even number of blocks, 64 to 126.
inline bool moe_packed_takes(int64_t k) {
  const int64_t nb = k / 32;
  return nb % 2 == 0 && nb >= 64 && nb <= 126;
}

// The streaming form's LDS: the chunk's activation rows and the waves' stage buffers.
inline bool moe_stream_fits(int64_t k) {
  const int64_t nb = k / 32;
  return k / 16 <= 64 * kMoeActLoads && nb <= 64 * kMoeScaleLoads &&
         ((size_t)kMoePairs * (k + nb * 4) + 15) / 16 * 16 + (size_t)kMoeSWaves * kStageBytes <= 160 * 1024;
}

template <int FMT>
hipError_t launch_moe_fmt(const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                          const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                          float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
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

bool moe_supported(int type, int64_t k) {
  return type == T_Q8_0 || type == T_IQ4_NL || type == T_MXFP4 || moe_kq_supported(type, k);
}

int moe_act_layout(int type) { return type == T_Q4_K || type == T_Q6_K ? ACT_Q8K : ACT_Q8_0; }

size_t moe_runs_bytes(int64_t size_m) { return (size_t)(1 + 3 * size_m) * sizeof(int32_t); }

hipError_t launch_moe(int type, const void* w, int num_experts, int64_t n, int64_t k, const ActPlanes& p,
                      const int32_t* runs, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                      float* dst, int64_t ldd, int cus, hipStream_t st) {
  if (type == T_MXFP4 && moe_fp4_takes(k))
    return launch_moe_fp4(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
  if (moe_stream_fits(k) && moe_packed_takes(k)) {
    switch (type) {
      case T_Q8_0: return launch_moe_f<T_Q8_0>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
      case T_IQ4_NL: return launch_moe_f<T_IQ4_NL>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
      case T_MXFP4: return launch_moe_f<T_MXFP4>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, st);
      default: return hipErrorInvalidValue;
    }
  }
  if (moe_stream_fits(k)) {
    switch (type) {
      case T_Q8_0: return launch_moe_s<T_Q8_0>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
      case T_IQ4_NL:
        return launch_moe_s<T_IQ4_NL>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
      case T_MXFP4: return launch_moe_s<T_MXFP4>(w, num_experts, n, k, p, runs, ids, topk_w, topk, size_m, dst, ldd, cus, st);
      default: return hipErrorInvalidValue;
    }
  }
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
