// matvec.hip — fused dequant + dot products for decode (1 activation row)
// and small-batch verification (2..8 rows) on gfx950.
//
// dst[r][row] = sum over the weight row's blocks of the block dot against
// activation row r, the arithmetic of candle's vec_dot per type
// (vendor/candle/candle-core/src/quantized/k_quants.rs: Q4_K 2031-2111,
// Q6_K 2598-2655, Q8_0 1294-1312, MXFP4 517-527, IQ4_NL 754-764) with
// exact int32 inner sums (v_dot4_i32_i8) and f32 scaling; only the f32
// summation order differs from the CPU's.
//
// Weights are read in GGUF bytes. The activation comes in the planes of
// qmm_launch.h (codes / scales / group sums, 16-byte aligned).
#include "b32_common.h"

namespace qmm {

constexpr int kWavesPerBlock = 4;

// ===========================================================================
// Q4_K: 144-byte super-blocks are 16-byte aligned, so each lane reads its
// part straight into registers. Lane = (super-block sb = lane/4 + 16t,
// 64-value chunk j = lane%4); a wave takes RPW weight rows and applies each
// lane's unpacked chunk to all NR activation rows.
// ===========================================================================
template <int NR, int RPW>
__global__ __launch_bounds__(256) void mv_q4k_kernel(const uint8_t* __restrict__ W, int64_t n, int nsb,
                                                     const int8_t* __restrict__ yq, const float* __restrict__ yd,
                                                     const int16_t* __restrict__ ybs, float* __restrict__ dst,
                                                     int64_t ldd) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * RPW;
  if (row0 >= n) return;
  const int j = lane & 3;
  const int64_t k = (int64_t)nsb * 256;
  const int64_t rb = (int64_t)nsb * 144;
  float acc[NR][RPW];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[r][i] = 0.0f;

  for (int sb = lane >> 2; sb < nsb; sb += 16) {
    uint4 hdr[RPW], qa[RPW], qb[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int64_t row = row0 + i < n ? row0 + i : n - 1;  // past the end: re-read, never written
      const uint8_t* blk = W + row * rb + (int64_t)sb * 144;
      hdr[i] = *(const uint4*)blk;
      qa[i] = *(const uint4*)(blk + 16 + 32 * j);
      qb[i] = *(const uint4*)(blk + 32 + 32 * j);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const int4* yp = (const int4*)(yq + r * k + (int64_t)sb * 256 + 64 * j);
      int yv[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int4 v = yp[q];
        yv[4 * q] = v.x; yv[4 * q + 1] = v.y; yv[4 * q + 2] = v.z; yv[4 * q + 3] = v.w;
      }
      const float dy = yd[r * nsb + sb];
      const int2 bb = *(const int2*)(ybs + (r * nsb + sb) * 16 + 4 * j);
      const int p0 = (int)(int16_t)(bb.x & 0xFFFF) + (int)(int16_t)((uint32_t)bb.x >> 16);
      const int p1 = (int)(int16_t)(bb.y & 0xFFFF) + (int)(int16_t)((uint32_t)bb.y >> 16);
#pragma unroll
      for (int i = 0; i < RPW; i++) acc[r][i] = q4k_unit(hdr[i], qa[i], qb[i], yv, dy, p0, p1, j, acc[r][i]);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const float v = wave_sum_dpp(acc[r][i]);
      if (lane == 0 && row0 + i < n) dst[r * ldd + row0 + i] = v;
    }
}

// ===========================================================================
// Q6_K from LDS. Lane = (super-block sb = lane/4 within the span, unit u =
// lane%4: half h = u/2, l0 = 16*(u%2)): the 64 values 128h + l0 + 32t +
// [0,16), t = 0..3, each group t with its own int8 scale.
// ===========================================================================
template <int NR, int RPW>
__global__ __launch_bounds__(256) void mv_q6k_kernel(const uint8_t* __restrict__ W, int64_t n, int nsb,
                                                     const int8_t* __restrict__ yq, const float* __restrict__ yd,
                                                     const int16_t* __restrict__ ybs, float* __restrict__ dst,
                                                     int64_t ldd) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kWavesPerBlock][RPW][kStageBytes];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * kWavesPerBlock + wv) * RPW;
  if (row0 >= n) return;
  const int64_t k = (int64_t)nsb * 256;
  const int64_t rb = (int64_t)nsb * 210;
  const int u = lane & 3, h = u >> 1, l0 = 16 * (u & 1);
  // per span of 16 super-blocks: one partial sum per (activation row, weight
  // row), the partials added in span order (the arithmetic of the streaming
  // kernel, which gives each span to its own wave)
  float tot[NR][RPW];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++) tot[r][i] = 0.0f;

  for (int s0 = 0; s0 < nsb; s0 += 16) {
    float acc[NR][RPW];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
      for (int i = 0; i < RPW; i++) acc[r][i] = 0.0f;
    const int nspan = nsb - s0 < 16 ? nsb - s0 : 16;
    int off[RPW];
    wave_lds_sync();  // the previous span's reads are done
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int64_t row = row0 + i < n ? row0 + i : n - 1;
      off[i] = stage_span(W, row * rb + (int64_t)s0 * 210, nspan * 210, smem[wv][i], lane);
    }
    wave_lds_sync();
    const int sbl = lane >> 2;
    if (sbl < nspan) {
      const int sb = s0 + sbl;
      // weight fields of this unit, per row
      uint32_t qlA[RPW][4], qlB[RPW][4], qh[RPW][4];
      int sc[RPW][4];
      float dx[RPW];
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        const uint8_t* L = smem[wv][i];
        const int b = off[i] + 210 * sbl;
        lds_words<4>(L, b + 64 * h + l0, qlA[i]);
        lds_words<4>(L, b + 64 * h + 32 + l0, qlB[i]);
        lds_words<4>(L, b + 128 + 32 * h + l0, qh[i]);
        uint32_t s4[2];
        lds_words<2>(L, b + 192 + 8 * h, s4);  // scales 8h .. 8h+7
        const int base = l0 >> 4;               // groups base, base+2, base+4, base+6
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int g = base + 2 * t;
          sc[i][t] = (int)(int8_t)((s4[g >> 2] >> (8 * (g & 3))) & 0xFF);
        }
        dx[i] = h2f((uint16_t)lds_u16(L, b + 208));
      }
#pragma unroll
      for (int r = 0; r < NR; r++) {
        const int8_t* yrow = yq + r * k + (int64_t)sb * 256 + 128 * h + l0;
        int yv[4][4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int4 q = *(const int4*)(yrow + 32 * t);
          yv[t][0] = q.x; yv[t][1] = q.y; yv[t][2] = q.z; yv[t][3] = q.w;
        }
        const float dy = yd[r * nsb + sb];
        const int4 bq = *(const int4*)(ybs + (r * nsb + sb) * 16 + 8 * h);  // bsums 8h .. 8h+7
        const uint32_t bw[4] = {(uint32_t)bq.x, (uint32_t)bq.y, (uint32_t)bq.z, (uint32_t)bq.w};
        const int bsh = 16 * (l0 >> 4);
        int bs[4];
#pragma unroll
        for (int t = 0; t < 4; t++) bs[t] = (int)(int16_t)((bw[t] >> bsh) & 0xFFFF);
#pragma unroll
        for (int i = 0; i < RPW; i++) acc[r][i] = q6k_unit(qlA[i], qlB[i], qh[i], sc[i], dx[i], yv, dy, bs, acc[r][i]);
      }
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        const float p = wave_sum_dpp(acc[r][i]);
        tot[r][i] = s0 == 0 ? p : __fadd_rn(tot[r][i], p);
      }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++)
      if (lane == 0 && row0 + i < n) dst[r * ldd + row0 + i] = tot[r][i];
}

// ===========================================================================
// 32-value formats (Q8_0, MXFP4, IQ4_NL) from LDS. Lane = unit of two
// blocks (64 values); a span is 128 blocks. Decode and per-unit arithmetic:
// b32_common.h.
// ===========================================================================
template <int FMT, int NR, int RPW>
__global__ __launch_bounds__(256) void mv_b32_kernel(const uint8_t* __restrict__ W, int64_t n, int nb,
                                                     const int8_t* __restrict__ yq, const float* __restrict__ yd,
                                                     float* __restrict__ dst, int64_t ldd) {
  using F = Fmt32<FMT>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kWavesPerBlock][RPW][kStageBytes];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * kWavesPerBlock + wv) * RPW;
  if (row0 >= n) return;
  const int64_t k = (int64_t)nb * 32;
  const int64_t rb = (int64_t)nb * F::B;
  const Lut32<FMT> lut;
  const uint32_t t0 = lut.t0, t1 = lut.t1, t2 = lut.t2, t3 = lut.t3;
  float acc[NR][RPW];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[r][i] = 0.0f;

  for (int b0 = 0; b0 < nb; b0 += 128) {
    const int nspan = nb - b0 < 128 ? nb - b0 : 128;
    int off[RPW];
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int64_t row = row0 + i < n ? row0 + i : n - 1;
      off[i] = stage_span(W, row * rb + (int64_t)b0 * F::B, nspan * F::B, smem[wv][i], lane);
    }
    wave_lds_sync();
    const int bl = 2 * lane;  // first block of this lane's unit, within the span
    if (bl < nspan) {
      const bool two = bl + 1 < nspan;
      uint32_t q[RPW][2][8];
      float dx[RPW][2];
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        F::decode(smem[wv][i], off[i] + bl * F::B, q[i][0], dx[i][0], t0, t1, t2, t3);
        if (two) {
          F::decode(smem[wv][i], off[i] + (bl + 1) * F::B, q[i][1], dx[i][1], t0, t1, t2, t3);
        } else {
#pragma unroll
          for (int t = 0; t < 8; t++) q[i][1][t] = 0;
          dx[i][1] = 0.0f;
        }
      }
      const int64_t gb = b0 + bl;  // global block index within the row
#pragma unroll
      for (int r = 0; r < NR; r++) {
        Act64 av;
        load_act64(av, yq, yd, r, k, nb, gb, two);
#pragma unroll
        for (int i = 0; i < RPW; i++) acc[r][i] = b32_unit(q[i][0], q[i][1], dx[i][0], dx[i][1], av, acc[r][i]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const float v = wave_sum_dpp(acc[r][i]);
      if (lane == 0 && row0 + i < n) dst[r * ldd + row0 + i] = v;
    }
}

// ===========================================================================
// dispatch
// ===========================================================================
int matvec_max_rows() { return 8; }

template <int NR>
static hipError_t launch_nr(int type, const void* w, int64_t n, int64_t k, const ActPlanes& p, float* dst,
                            int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const uint8_t* W = (const uint8_t*)w;
  if (type == T_Q4_K || type == T_Q6_K) {
    const int nsb = (int)(k / 256);
    if (type == T_Q4_K) {
      constexpr int RPW = NR <= 2 ? 4 : 2;
      const int64_t waves = (n + RPW - 1) / RPW;
      mv_q4k_kernel<NR, RPW><<<dim3((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock)), 256, 0, st>>>(
          W, n, nsb, p.codes, p.d, (const int16_t*)p.sums, dst, ldd);
    } else {
      constexpr int RPW = NR <= 2 ? 2 : 1;
      const int64_t waves = (n + RPW - 1) / RPW;
      mv_q6k_kernel<NR, RPW><<<dim3((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock)), 256, 0, st>>>(
          W, n, nsb, p.codes, p.d, (const int16_t*)p.sums, dst, ldd);
    }
    return hipGetLastError();
  }
  const int nb = (int)(k / 32);
  constexpr int RPW = NR <= 2 ? 2 : 1;
  const int64_t waves = (n + RPW - 1) / RPW;
  const dim3 grid((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock));
  switch (type) {
    case T_Q8_0: mv_b32_kernel<T_Q8_0, NR, RPW><<<grid, 256, 0, st>>>(W, n, nb, p.codes, p.d, dst, ldd); break;
    case T_IQ4_NL: mv_b32_kernel<T_IQ4_NL, NR, RPW><<<grid, 256, 0, st>>>(W, n, nb, p.codes, p.d, dst, ldd); break;
    case T_MXFP4: mv_b32_kernel<T_MXFP4, NR, RPW><<<grid, 256, 0, st>>>(W, n, nb, p.codes, p.d, dst, ldd); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_matvec(int type, const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                         int64_t ldd, hipStream_t st) {
  switch (rows) {
    case 1: return launch_nr<1>(type, w, n, k, p, dst, ldd, st);
    case 2: return launch_nr<2>(type, w, n, k, p, dst, ldd, st);
    case 3: return launch_nr<3>(type, w, n, k, p, dst, ldd, st);
    case 4: return launch_nr<4>(type, w, n, k, p, dst, ldd, st);
    case 5: return launch_nr<5>(type, w, n, k, p, dst, ldd, st);
    case 6: return launch_nr<6>(type, w, n, k, p, dst, ldd, st);
    case 7: return launch_nr<7>(type, w, n, k, p, dst, ldd, st);
    case 8: return launch_nr<8>(type, w, n, k, p, dst, ldd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qmm
