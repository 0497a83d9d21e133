// mv_q4k.hip — Q4_K decode matvec (1-2 activation rows) for gfx950.
//
// Arithmetic: candle's Q4_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2031-2111):
//   per super-block  d*dy * sum_j sc_j * sum_{32} q*y  -  dmin*dy * sum_j m_j * (bsum_2j + bsum_2j+1)
// with every inner sum an exact int32 (v_dot4_i32_i8) and f32 scaling.
//
// Shape of the work: a streaming kernel. Each wave walks weight rows
// gw, gw + W, gw + 2W, ... (gw its index among the W waves of the grid) and
// (with PF) keeps the next row's loads in flight while it computes one, so
// the VALU work of a row runs under the transfer of the next instead of
// piling up after the last byte lands (a kernel that loads everything first
// and computes after spends that compute as a tail: ~1.7 us per SIMD for a
// 33 MB Q4_K matrix at 4 cycles per wave64 instruction).
//
// Lane L of a wave owns the 64-value unit (super-block sb = L/4 + 16t,
// chunk j = L%4: sub-blocks 2j, 2j+1) of every row, so its slice of the
// activation is the same for every row and lives in registers: the
// workgroup quantizes the f32 activation into LDS once (FUSED; the codes,
// scales and group sums of BlockQ8K::from_float bit for bit, through the
// q8k_block_group16 the standalone quantizer runs) or copies pre-quantized
// planes there, and each lane then takes its slice. Per row a lane loads the
// 16-byte header and its 32 code bytes of each of its super-blocks.
//
// One launch may cover up to kMaxTargets weights of the same k that share
// the activation (QMatMul::forward_shared, quantized/mod.rs:1221-1263): the
// rows of the targets are numbered one after another.
#include "glu_act.h"
#include "mv_common.h"

namespace qmm {

namespace {


// A row's bytes for one lane: per super-block t, the header and the 32 code bytes of chunk j.
template <int T>
struct RowRegs {
  uint4 h[T], qa[T], qb[T];
};

template <int T>
__device__ __forceinline__ void load_row(RowRegs<T>& rr, const uint8_t* __restrict__ row, int nsb, int lane) {
  const int j = lane & 3, sbl = lane >> 2;
#pragma unroll
  for (int t = 0; t < T; t++) {
    const int sb = sbl + 16 * t;
    if (sb < nsb) {
      const uint8_t* blk = row + sb * 144;
      rr.h[t] = *(const uint4*)blk;
      rr.qa[t] = *(const uint4*)(blk + 16 + 32 * j);
      rr.qb[t] = *(const uint4*)(blk + 32 + 32 * j);
    } else {
      rr.h[t] = rr.qa[t] = rr.qb[t] = make_uint4(0, 0, 0, 0);
    }
  }
}

// The row as contiguous 16-byte pieces: lane L holds pieces L + 64c. Each
// byte is loaded once, by one lane, so the loads can take the nontemporal
// hint; a wave-private LDS slot then turns them into the per-lane layout of
// RowRegs (unpack_row).
template <int T>
struct RowRaw {
  static constexpr int kLoads = (9 * 16 * T + 63) / 64;  // 9 pieces per super-block
  uint4 p[kLoads];
};

template <int T>
__device__ __forceinline__ void load_raw(RowRaw<T>& rr, const uint8_t* __restrict__ row, int nsb, int lane) {
  const int pieces = 9 * nsb;
#pragma unroll
  for (int c = 0; c < RowRaw<T>::kLoads; c++) {
    const int pc = lane + 64 * c;
    rr.p[c] = pc < pieces ? ld_stream16(row + 16 * pc) : make_uint4(0, 0, 0, 0);
  }
}

// Writes the row's pieces to the wave's LDS slot and reads back the header and
// code bytes of this lane's units. The next row's writes reach the slot after
// these reads: LDS operations of one wave complete in order.
template <int T>
__device__ __forceinline__ void unpack_row(const RowRaw<T>& rr, uint8_t* slot, RowRegs<T>& out, int nsb, int lane) {
  const int pieces = 9 * nsb;
#pragma unroll
  for (int c = 0; c < RowRaw<T>::kLoads; c++) {
    const int pc = lane + 64 * c;
    if (pc < pieces) *(uint4*)(slot + 16 * pc) = rr.p[c];
  }
  wave_lds_sync();
  const int j = lane & 3, sbl = lane >> 2;
#pragma unroll
  for (int t = 0; t < T; t++) {
    const int sb = sbl + 16 * t;
    if (sb < nsb) {
      const uint8_t* blk = slot + sb * 144;
      out.h[t] = *(const uint4*)blk;
      out.qa[t] = *(const uint4*)(blk + 16 + 32 * j);
      out.qb[t] = *(const uint4*)(blk + 32 + 32 * j);
    } else {
      out.h[t] = out.qa[t] = out.qb[t] = make_uint4(0, 0, 0, 0);
    }
  }
}

// A lane's slice of one activation row: the 64 codes of its unit per
// super-block t, dy, and the code sums of sub-blocks 2j, 2j+1.
template <int T>
struct ActRegs {
  int y[T][16];
  float dy[T];
  int32_t p0[T], p1[T];
};

// Rows of up to 4096 values (T == 1) hold 8 waves a SIMD (two 16-wave
// workgroups a CU, 64 registers a lane): the grid of the largest products
// (gate+up) is sized for that.
template <int NR, int T, bool FUSED, int kWaves, bool PF, bool XCHG>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(T == 1 && NR == 1 ? 8 : 1)))
void mv_q4k_stream_kernel(MvTargets tg, int nsb, const float* __restrict__ x,
                                                            int64_t xstride, const int8_t* __restrict__ yq,
                                                            const float* __restrict__ yd,
                                                            const int16_t* __restrict__ ybs, float qmax) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const ActLds s = act_lds(smem, NR, nsb);

  // the wave index is uniform: rows, targets and pointers stay scalar
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 3, sbl = lane >> 2;
  const int k = nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;
  const int64_t n_total = tg.row_end[tg.count - 1];
  // workgroup b owns rows [b N / G, (b + 1) N / G), its waves interleaved
  // within: every CU streams the same number of rows (a stride over the whole
  // grid leaves the CUs that host two workgroups of full waves a row in 7
  // more: 14336 rows over 8192 waves, 64 against 48 rows a CU)
  const int64_t G = gridDim.x;
  const int64_t gw = (int64_t)blockIdx.x * n_total / G + wv;
  const int64_t R_end = (int64_t)(blockIdx.x + 1) * n_total / G;
  constexpr int64_t W = kWaves;

  auto row_ptr = [&](int64_t R, float*& out, int64_t& ldd) -> const uint8_t* {
    int t = 0;
#pragma unroll
    for (int i = 0; i < kMaxTargets - 1; i++)
      if (i < tg.count - 1 && R >= tg.row_end[i]) t = i + 1;
    const int64_t lrow = R - (t ? tg.row_end[t - 1] : 0);
    out = tg.dst[t] + lrow;
    ldd = tg.ldd[t];
    return (const uint8_t*)tg.w[t] + lrow * rowbytes;
  };

  // XCHG: the wave's LDS slot for unpacking contiguous row loads, after the activation
  uint8_t* slot = smem + act_lds_bytes(NR, nsb) + (size_t)wv * 144 * nsb;

  // 1. activation loads, then the first row's weight loads
  ActBatch<NR, FUSED, kWaves> act;
  act.load(nsb, x, xstride, yq, yd, ybs);
  RowRegs<T> cur;
  RowRaw<T> craw;
  float* out = nullptr;
  int64_t ldd = 0;
  if (gw < R_end) {
    if (XCHG)
      load_raw<T>(craw, row_ptr(gw, out, ldd), nsb, lane);
    else
      load_row<T>(cur, row_ptr(gw, out, ldd), nsb, lane);
  }

  // 2. the activation into LDS, then each lane's slice into registers
  act.store(s, nsb, x, xstride, yq, yd, ybs, qmax);
  __syncthreads();
  ActRegs<T> a[NR];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int sb = sbl + 16 * t;
      if (sb < nsb) {
        const int4* yp = (const int4*)(s.codes + r * k + sb * 256 + 64 * j);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int4 v = yp[q];
          a[r].y[t][4 * q] = v.x; a[r].y[t][4 * q + 1] = v.y; a[r].y[t][4 * q + 2] = v.z; a[r].y[t][4 * q + 3] = v.w;
        }
        a[r].dy[t] = s.dy[r * nsb + sb];
        const int32_t* g = s.s16 + (r * nsb + sb) * 16 + 4 * j;  // sub-blocks 2j, 2j+1 = groups 4j .. 4j+3
        a[r].p0[t] = g[0] + g[1];
        a[r].p1[t] = g[2] + g[3];
      } else {
#pragma unroll
        for (int q = 0; q < 16; q++) a[r].y[t][q] = 0;
        a[r].dy[t] = 0.0f;
        a[r].p0[t] = a[r].p1[t] = 0;
      }
    }

  // 3. stream the rows. The results of a wave's first two rows are stored
  // when its rows are done: a store in the loop would hold the wait for the
  // next row's loads until the store is acknowledged (a wave's loads and
  // stores share one counter; 0.3-0.5 us on C2's gate).
  float keep0[NR], keep1[NR];
  float* kout0 = nullptr;
  float* kout1 = nullptr;
  int64_t kldd0 = 0, kldd1 = 0;
  int done = 0;
  for (int64_t R = gw; R < R_end; R += W) {
    // PF: the next row's loads go out before this row's compute
    RowRegs<T> nxt;
    RowRaw<T> nraw;
    float* nout = nullptr;
    int64_t nldd = 0;
    if (PF && R + W < R_end) {
      if (XCHG)
        load_raw<T>(nraw, row_ptr(R + W, nout, nldd), nsb, lane);
      else
        load_row<T>(nxt, row_ptr(R + W, nout, nldd), nsb, lane);
    }
    if (XCHG) unpack_row<T>(craw, slot, cur, nsb, lane);

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int r = 0; r < NR; r++)
        acc[r] = q4k_unit(cur.h[t], cur.qa[t], cur.qb[t], a[r].y[t], a[r].dy[t], a[r].p0[t], a[r].p1[t], j, acc[r]);
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const float v = wave_sum_dpp(acc[r]);
      if (done == 0) {
        keep0[r] = v;
      } else if (done == 1) {
        keep1[r] = v;
      } else if (lane == 0) {
        out[r * ldd] = v;
      }
    }
    if (done == 0) {
      kout0 = out;
      kldd0 = ldd;
    } else if (done == 1) {
      kout1 = out;
      kldd1 = ldd;
    }
    done++;
    if (PF) {
      if (XCHG)
        craw = nraw;
      else
        cur = nxt;
      out = nout;
      ldd = nldd;
    } else if (R + W < R_end) {
      if (XCHG)
        load_raw<T>(craw, row_ptr(R + W, out, ldd), nsb, lane);
      else
        load_row<T>(cur, row_ptr(R + W, out, ldd), nsb, lane);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < NR; r++) {
      if (done > 0) kout0[r * kldd0] = keep0[r];
      if (done > 1) kout1[r * kldd1] = keep1[r];
    }
  }
}

// Rows are unpacked through LDS (contiguous nontemporal loads) up to 4096
// values a row, where two 16-wave workgroups' slots (36 KB each) still fit a
// CU beside their activations.
inline bool q4k_xchg(int nsb) { return nsb <= 16; }

template <int NR, int T, int WPG, bool PF, bool XCHG>
hipError_t launch_stream_x(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                           float qmax, int64_t waves, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const size_t lds = act_lds_bytes(NR, nsb) + (XCHG ? (size_t)WPG * 144 * nsb : 0);
  const dim3 grid((unsigned)((waves + WPG - 1) / WPG));
  if (pre) {
    constexpr auto* k = &mv_q4k_stream_kernel<NR, T, false, WPG, PF, XCHG>;
    if (lds > 65536 && set_max_dynamic_lds<k>() != hipSuccess) return hipErrorInvalidValue;
    k<<<grid, 64 * WPG, lds, st>>>(t, nsb, nullptr, 0, pre->codes, pre->d, (const int16_t*)pre->sums, qmax);
  } else {
    constexpr auto* k = &mv_q4k_stream_kernel<NR, T, true, WPG, PF, XCHG>;
    if (lds > 65536 && set_max_dynamic_lds<k>() != hipSuccess) return hipErrorInvalidValue;
    k<<<grid, 64 * WPG, lds, st>>>(t, nsb, x, xstride, nullptr, nullptr, nullptr, qmax);
  }
  return hipGetLastError();
}

template <int NR, int T, int WPG, bool PF>
hipError_t launch_stream(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                         float qmax, int64_t waves, hipStream_t st) {
  if (T <= 2 && q4k_xchg(nsb)) return launch_stream_x<NR, T, WPG, PF, true>(t, nsb, x, xstride, pre, qmax, waves, st);
  return launch_stream_x<NR, T, WPG, PF, false>(t, nsb, x, xstride, pre, qmax, waves, st);
}

template <int NR, int T>
hipError_t launch_shape(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                        float qmax, const MvShape& sh, hipStream_t st) {
  if (sh.wpg == 16)
    return sh.prefetch ? launch_stream<NR, T, 16, true>(t, nsb, x, xstride, pre, qmax, sh.waves, st)
                       : launch_stream<NR, T, 16, false>(t, nsb, x, xstride, pre, qmax, sh.waves, st);
  return sh.prefetch ? launch_stream<NR, T, 4, true>(t, nsb, x, xstride, pre, qmax, sh.waves, st)
                     : launch_stream<NR, T, 4, false>(t, nsb, x, xstride, pre, qmax, sh.waves, st);
}

// The gate and up products of an MLP and the GLU between them in one
// launch (the reference's forward_shared of ffn_up and ffn_gate followed by
// silu_mul / swiglu_oai_mul / gelu, src/inference/layers/mod.rs:583-632):
// the stream kernel above with a unit of two weight rows, gate row j and up
// row j, which one wave computes against the shared activation before lane 0
// writes act(g) * u. Both rows are unpacked through the wave's LDS slot in
// turn; with PF the next pair's loads are in flight under the current pair.
template <int NR, int T, bool FUSED, int kWaves, bool PF, int ACT>
__global__ __launch_bounds__(64 * kWaves) void mv_q4k_glu_kernel(const uint8_t* __restrict__ wg,
                                                                 const uint8_t* __restrict__ wu, int64_t n, int nsb,
                                                                 const float* __restrict__ x, int64_t xstride,
                                                                 const int8_t* __restrict__ yq,
                                                                 const float* __restrict__ yd,
                                                                 const int16_t* __restrict__ ybs, float qmax,
                                                                 float* __restrict__ dst, int64_t ldd) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const ActLds s = act_lds(smem, NR, nsb);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 3, sbl = lane >> 2;
  const int k = nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;
  const int64_t W = (int64_t)gridDim.x * kWaves;
  const int64_t gw = (int64_t)blockIdx.x * kWaves + wv;
  uint8_t* slot = smem + act_lds_bytes(NR, nsb) + (size_t)wv * 144 * nsb;

  ActBatch<NR, FUSED, kWaves> act;
  act.load(nsb, x, xstride, yq, yd, ybs);
  RowRaw<T> cg, cu;
  if (gw < n) {
    load_raw<T>(cg, wg + gw * rowbytes, nsb, lane);
    load_raw<T>(cu, wu + gw * rowbytes, nsb, lane);
  }
  act.store(s, nsb, x, xstride, yq, yd, ybs, qmax);
  __syncthreads();
  ActRegs<T> a[NR];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int sb = sbl + 16 * t;
      if (sb < nsb) {
        const int4* yp = (const int4*)(s.codes + r * k + sb * 256 + 64 * j);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int4 v = yp[q];
          a[r].y[t][4 * q] = v.x; a[r].y[t][4 * q + 1] = v.y; a[r].y[t][4 * q + 2] = v.z; a[r].y[t][4 * q + 3] = v.w;
        }
        a[r].dy[t] = s.dy[r * nsb + sb];
        const int32_t* g = s.s16 + (r * nsb + sb) * 16 + 4 * j;
        a[r].p0[t] = g[0] + g[1];
        a[r].p1[t] = g[2] + g[3];
      } else {
#pragma unroll
        for (int q = 0; q < 16; q++) a[r].y[t][q] = 0;
        a[r].dy[t] = 0.0f;
        a[r].p0[t] = a[r].p1[t] = 0;
      }
    }

  for (int64_t R = gw; R < n; R += W) {
    RowRaw<T> ng, nu;
    if (PF && R + W < n) {
      load_raw<T>(ng, wg + (R + W) * rowbytes, nsb, lane);
      load_raw<T>(nu, wu + (R + W) * rowbytes, nsb, lane);
    }
    float ag[NR], au[NR];
    {
      RowRegs<T> rr;
      unpack_row<T>(cg, slot, rr, nsb, lane);
#pragma unroll
      for (int r = 0; r < NR; r++) ag[r] = 0.0f;
#pragma unroll
      for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < NR; r++)
          ag[r] = q4k_unit(rr.h[t], rr.qa[t], rr.qb[t], a[r].y[t], a[r].dy[t], a[r].p0[t], a[r].p1[t], j, ag[r]);
    }
    {
      // the slot's second use: the gate row's reads above complete first
      RowRegs<T> rr;
      unpack_row<T>(cu, slot, rr, nsb, lane);
#pragma unroll
      for (int r = 0; r < NR; r++) au[r] = 0.0f;
#pragma unroll
      for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < NR; r++)
          au[r] = q4k_unit(rr.h[t], rr.qa[t], rr.qb[t], a[r].y[t], a[r].dy[t], a[r].p0[t], a[r].p1[t], j, au[r]);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const float g = wave_sum_dpp(ag[r]);
      const float u = wave_sum_dpp(au[r]);
      if (lane == 0) dst[r * ldd + R] = glu_act<ACT>(g, u);
    }
    if (PF) {
      cg = ng;
      cu = nu;
    } else if (R + W < n) {
      load_raw<T>(cg, wg + (R + W) * rowbytes, nsb, lane);
      load_raw<T>(cu, wu + (R + W) * rowbytes, nsb, lane);
    }
  }
}

template <int NR, int T, bool PF, int ACT>
hipError_t launch_glu_x(const void* wg, const void* wu, int64_t n, int nsb, const float* x, int64_t xstride,
                        const ActPlanes* pre, float qmax, float* dst, int64_t ldd, int64_t waves, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  constexpr int WPG = 16;
  const size_t lds = act_lds_bytes(NR, nsb) + (size_t)WPG * 144 * nsb;
  const dim3 grid((unsigned)((waves + WPG - 1) / WPG));
  if (pre) {
    constexpr auto* kf = &mv_q4k_glu_kernel<NR, T, false, WPG, PF, ACT>;
    if (lds > 65536 && set_max_dynamic_lds<kf>() != hipSuccess) return hipErrorInvalidValue;
    kf<<<grid, 64 * WPG, lds, st>>>((const uint8_t*)wg, (const uint8_t*)wu, n, nsb, nullptr, 0, pre->codes, pre->d,
                                    (const int16_t*)pre->sums, qmax, dst, ldd);
  } else {
    constexpr auto* kf = &mv_q4k_glu_kernel<NR, T, true, WPG, PF, ACT>;
    if (lds > 65536 && set_max_dynamic_lds<kf>() != hipSuccess) return hipErrorInvalidValue;
    kf<<<grid, 64 * WPG, lds, st>>>((const uint8_t*)wg, (const uint8_t*)wu, n, nsb, x, xstride, nullptr, nullptr,
                                    nullptr, qmax, dst, ldd);
  }
  return hipGetLastError();
}

template <int NR, int T, int ACT>
hipError_t launch_glu_pf(const void* wg, const void* wu, int64_t n, int nsb, const float* x, int64_t xstride,
                         const ActPlanes* pre, float qmax, float* dst, int64_t ldd, int cus, hipStream_t st) {
  // one 16-wave workgroup a CU; a pair a wave where pairs are few, else the
  // pairs spread over the CUs with the next pair in flight (C2's 14336 pairs:
  // 14.6 us; two workgroups a CU 15.9 us, a pair a wave 20.2 us)
  const int64_t cap = (int64_t)cus * 16;
  if (n <= cap)
    return launch_glu_x<NR, T, false, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, (n + 15) / 16 * 16, st);
  return launch_glu_x<NR, T, true, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, cap, st);
}

template <int ACT>
hipError_t launch_glu_act(const void* wg, const void* wu, int64_t n, int nsb, int64_t rows, const float* x,
                          int64_t xstride, const ActPlanes* pre, float qmax, float* dst, int64_t ldd, int cus,
                          hipStream_t st) {
  const int T = (nsb + 15) / 16;
  if (rows == 1)
    return T <= 1 ? launch_glu_pf<1, 1, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, cus, st)
                  : launch_glu_pf<1, 2, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, cus, st);
  return T <= 1 ? launch_glu_pf<2, 1, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, cus, st)
                : launch_glu_pf<2, 2, ACT>(wg, wu, n, nsb, x, xstride, pre, qmax, dst, ldd, cus, st);
}

}  // namespace

bool mv_q4k_rows_supported(int64_t k, int64_t rows) {
  return rows >= 1 && rows <= 2 && k % 256 == 0 && k >= 256 && k <= (rows == 1 ? 16384 : 8192);
}

bool mv_q4k_rows_fusable(const float* x, int64_t xstride) {
  return ((uintptr_t)x & 15) == 0 && xstride % 4 == 0;
}

// Waves in the grid: each wave streams about `per_wave` weight rows.
int64_t mv_q4k_rows_waves(int64_t n_total, int per_wave) {
  const int64_t w = (n_total + per_wave - 1) / per_wave;
  return (w + 15) / 16 * 16;
}

hipError_t launch_mv_q4k_rows(const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, float qmax, const MvShape& sh, hipStream_t st) {
  const int nsb = (int)(k / 256);
  const int T = (nsb + 15) / 16;
  if (rows == 1) {
    if (T <= 1) return launch_shape<1, 1>(t, nsb, x, xstride, pre, qmax, sh, st);
    if (T <= 2) return launch_shape<1, 2>(t, nsb, x, xstride, pre, qmax, sh, st);
    return launch_shape<1, 4>(t, nsb, x, xstride, pre, qmax, sh, st);
  }
  if (T <= 1) return launch_shape<2, 1>(t, nsb, x, xstride, pre, qmax, sh, st);
  return launch_shape<2, 2>(t, nsb, x, xstride, pre, qmax, sh, st);
}

// Rows of up to 8192 values (two units of 16 super-blocks a lane), 1-2
// activation rows: the fused gate+up+GLU launch.
bool mv_q4k_glu_supported(int64_t k, int64_t rows) {
  return rows >= 1 && rows <= 2 && k % 256 == 0 && k >= 256 && k <= 8192;
}

hipError_t launch_mv_q4k_glu(int act, const void* wg, const void* wu, int64_t n, int64_t k, int64_t rows,
                             const float* x, int64_t xstride, const ActPlanes* pre, float qmax, float* dst, int64_t ldd,
                             int cus, hipStream_t st) {
  const int nsb = (int)(k / 256);
  if (act == GLU_SILU) return launch_glu_act<GLU_SILU>(wg, wu, n, nsb, rows, x, xstride, pre, qmax, dst, ldd, cus, st);
  if (act == GLU_SWIGLU_OAI)
    return launch_glu_act<GLU_SWIGLU_OAI>(wg, wu, n, nsb, rows, x, xstride, pre, qmax, dst, ldd, cus, st);
  if (act == GLU_GELU) return launch_glu_act<GLU_GELU>(wg, wu, n, nsb, rows, x, xstride, pre, qmax, dst, ldd, cus, st);
  return hipErrorInvalidValue;
}

}  // namespace qmm
