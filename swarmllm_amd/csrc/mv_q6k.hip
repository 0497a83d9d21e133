// mv_q6k.hip — Q6_K decode matvec (1-2 activation rows) for gfx950.
//
// Arithmetic: candle's Q6_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2598-2655): per
// 16-value group, d*dy * sc_g * sum (q-32)*y with q the 6-bit code
// (ql nibble | qh 2 bits << 4); every inner sum an exact int32.
//
// A Q6_K super-block is 210 bytes, so blocks are not 16-byte aligned: a wave
// stages each span of 16 super-blocks of a row (3360 bytes, the loads 64
// consecutive 16-byte pieces per instruction) into its own LDS buffer and
// computes from there, one 64-value unit per lane (super-block sbl = L/4 of
// the span, unit u = L%4: half h = u/2, l0 = 16*(u%2)), through the same
// q6k_unit the multi-row kernel runs, and (PF) keeps its next span's loads in
// flight in registers while it computes the current one. The workgroup
// quantizes the f32 activation into LDS once (FUSED) or copies pre-quantized
// planes there.
//
// One launch may cover up to kMaxTargets weights of the same k sharing the
// activation (QMatMul::forward_shared, quantized/mod.rs:1221-1263).
#include "mv_common.h"

namespace qmm {

namespace {

constexpr int kSpanSb = 16;                            // super-blocks per span
constexpr int kSpanBytes = kSpanSb * 210;              // 3360
constexpr int kSpanPieces = (kSpanBytes + 15) / 16 + 1; // 16-byte pieces, start not aligned: 211
constexpr int kPiecesPerLane = (kSpanPieces + 63) / 64; // 4
// LDS bytes per wave: the pieces, and the 8 bytes past the last that the
// dword reads of lds_words may touch
constexpr int kSpanBuf = kSpanPieces * 16 + 16;

struct Span {
  uint4 p[kPiecesPerLane];
  int off;  // offset of the span's first byte in its first piece
  int len;  // super-blocks in the span
};

// Loads the 16-byte aligned pieces (aligned as device addresses) from the one
// holding byte p to the one holding byte p + len*210 - 1. Every piece read
// holds at least one byte of the span, and an aligned piece never crosses a
// page, so the bytes read beyond the span stay in mapped memory.
__device__ __forceinline__ void load_span(Span& sp, const uint8_t* __restrict__ p, int len, int lane) {
  // rounded down by pointer arithmetic: the compiler keeps these global
  // loads (an integer round trip would make them flat loads, which every LDS
  // wait also waits for)
  sp.off = (int)((uintptr_t)p & 15);
  const uint8_t* a0 = p - sp.off;
  sp.len = len;
  const int pieces = (int)((sp.off + len * 210 + 15) >> 4);
#pragma unroll
  for (int c = 0; c < kPiecesPerLane; c++) {
    const int pc = lane + 64 * c;
    sp.p[c] = pc < pieces ? ld_stream16(a0 + 16 * pc) : make_uint4(0, 0, 0, 0);
  }
}

// Work: the spans of a row go to different waves of one workgroup. With
// nspan spans per row, a workgroup of kWaves waves takes G = kWaves / nspan
// rows at a time: wave wv works span wv % nspan of row-slot wv / nspan. Each
// wave reduces its span's partial sum (wave_sum_dpp) into LDS; after the
// workgroup barrier the span-0 wave of each row-slot adds the partials in
// span order and writes the row. Row-slots walk the rows
// (blockIdx.x + i * gridDim.x) * G + g, every wave of the grid the same
// number of iterations (a wave without a row still meets the barriers).
template <int NR, bool FUSED, int kWaves, bool PF>
__global__ __launch_bounds__(64 * kWaves) void mv_q6k_stream_kernel(MvTargets tg, int nsb, const float* __restrict__ x,
                                                                    int64_t xstride, const int8_t* __restrict__ yq,
                                                                    const float* __restrict__ yd,
                                                                    const int16_t* __restrict__ ybs, float qmax) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const ActLds s = act_lds(smem, NR, nsb);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const part_base = smem + (act_lds_bytes(NR, nsb) + 15) / 16 * 16;  // [2][kWaves][NR] floats
  uint8_t* buf = part_base + 2 * kWaves * NR * 4 + (size_t)wv * kSpanBuf;
  float* const part = (float*)part_base;
  const int k = nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 210;
  const int64_t n_total = tg.row_end[tg.count - 1];
  const int nspan = (nsb + kSpanSb - 1) / kSpanSb;
  const int G = kWaves / nspan;  // rows per workgroup iteration
  const int g = wv / nspan, span = wv - g * nspan;
  const bool active = g < G;
  const int s0 = span * kSpanSb;
  const int len = nsb - s0 < kSpanSb ? nsb - s0 : kSpanSb;
  const int64_t rows_per_iter = (int64_t)gridDim.x * G;
  const int64_t iters = (n_total + rows_per_iter - 1) / rows_per_iter;

  auto row_of = [&](int64_t i) -> int64_t { return ((int64_t)blockIdx.x + i * gridDim.x) * G + g; };
  auto row_ptr = [&](int64_t R, float*& out, int64_t& ldd) -> const uint8_t* {
    int t = 0;
#pragma unroll
    for (int q = 0; q < kMaxTargets - 1; q++)
      if (q < tg.count - 1 && R >= tg.row_end[q]) t = q + 1;
    const int64_t lrow = R - (t ? tg.row_end[t - 1] : 0);
    out = tg.dst[t] + lrow;
    ldd = tg.ldd[t];
    return (const uint8_t*)tg.w[t] + lrow * rowbytes;
  };

  // 1. activation loads, then the first span's weight loads
  ActBatch<NR, FUSED, kWaves> act;
  act.load(nsb, x, xstride, yq, yd, ybs);
  Span cur;
  float* out = nullptr;
  int64_t ldd = 0;
  if (active && row_of(0) < n_total) load_span(cur, row_ptr(row_of(0), out, ldd) + (int64_t)s0 * 210, len, lane);

  // 2. the activation into LDS
  act.store(s, nsb, x, xstride, yq, yd, ybs, qmax);
  __syncthreads();

  // 3. stream the rows
  const int sbl = lane >> 2, u = lane & 3, h = u >> 1, l0 = 16 * (u & 1);
  for (int64_t i = 0; i < iters; i++) {
    const int64_t R = row_of(i);
    const bool have = active && R < n_total;
    float* cout = out;
    const int64_t cldd = ldd;
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.0f;
    Span nxt;
    if (have) {
      // the span into this wave's LDS buffer
      wave_lds_sync();  // the previous span's reads are done
#pragma unroll
      for (int c = 0; c < kPiecesPerLane; c++)
        if (lane + 64 * c < kSpanPieces) *(uint4*)(buf + 16 * (lane + 64 * c)) = cur.p[c];
      wave_lds_sync();
      const int off = cur.off;
      if (PF && row_of(i + 1) < n_total)
        load_span(nxt, row_ptr(row_of(i + 1), out, ldd) + (int64_t)s0 * 210, len, lane);
      if (sbl < len) {
        const int b = off + 210 * sbl;
        uint32_t qlA[4], qlB[4], qh[4], s4[2];
        lds_words<4>(buf, b + 64 * h + l0, qlA);
        lds_words<4>(buf, b + 64 * h + 32 + l0, qlB);
        lds_words<4>(buf, b + 128 + 32 * h + l0, qh);
        lds_words<2>(buf, b + 192 + 8 * h, s4);  // scales 8h .. 8h+7
        int sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int gg = (l0 >> 4) + 2 * t;
          sc[t] = (int)(int8_t)((s4[gg >> 2] >> (8 * (gg & 3))) & 0xFF);
        }
        const float dx = h2f((uint16_t)lds_u16(buf, b + 208));
        const int sb = s0 + sbl;
#pragma unroll
        for (int r = 0; r < NR; r++) {
          const int8_t* yrow = s.codes + r * k + sb * 256 + 128 * h + l0;
          int yv[4][4], bs[4];
#pragma unroll
          for (int t = 0; t < 4; t++) {
            const int4 q = *(const int4*)(yrow + 32 * t);
            yv[t][0] = q.x; yv[t][1] = q.y; yv[t][2] = q.z; yv[t][3] = q.w;
            bs[t] = s.s16[(r * nsb + sb) * 16 + 8 * h + 2 * t + (l0 >> 4)];
          }
          acc[r] = q6k_unit(qlA, qlB, qh, sc, dx, yv, s.dy[r * nsb + sb], bs, acc[r]);
        }
      }
    }
    // partial sums of the spans, added in span order
    float* slot = part + (i & 1) * kWaves * NR;
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const float v = wave_sum_dpp(acc[r]);
      if (lane == 0) slot[wv * NR + r] = v;
    }
    __syncthreads();
    if (have && span == 0 && lane == 0) {
#pragma unroll
      for (int r = 0; r < NR; r++) {
        float tot = slot[(g * nspan) * NR + r];
        for (int q = 1; q < nspan; q++) tot = __fadd_rn(tot, slot[(g * nspan + q) * NR + r]);
        cout[r * cldd] = tot;
      }
    }
    if (PF) {
      cur = nxt;
    } else if (active && row_of(i + 1) < n_total) {
      load_span(cur, row_ptr(row_of(i + 1), out, ldd) + (int64_t)s0 * 210, len, lane);
    }
  }
}

template <int NR, int WPG, bool PF>
size_t stream_lds(int nsb) {
  return (act_lds_bytes(NR, nsb) + 15) / 16 * 16 + 2 * WPG * NR * 4 + (size_t)WPG * kSpanBuf;
}

template <int NR, int WPG, bool PF>
hipError_t launch_stream(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                         float qmax, int64_t waves, hipStream_t st) {
  const size_t lds = stream_lds<NR, WPG, PF>(nsb);
  const dim3 grid((unsigned)((waves + WPG - 1) / WPG));
  // dynamic LDS past 64 KiB needs the kernel's limit raised (to the 160 KiB
  // of a CU), once per kernel
  static bool raised[2] = {false, false};
  if (pre) {
    auto* kfn = &mv_q6k_stream_kernel<NR, false, WPG, PF>;
    if (!raised[0]) {
      if (hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
        return hipErrorInvalidValue;
      raised[0] = true;
    }
    kfn<<<grid, 64 * WPG, lds, st>>>(t, nsb, nullptr, 0, pre->codes, pre->d, (const int16_t*)pre->sums, qmax);
  } else {
    auto* kfn = &mv_q6k_stream_kernel<NR, true, WPG, PF>;
    if (!raised[1]) {
      if (hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
        return hipErrorInvalidValue;
      raised[1] = true;
    }
    kfn<<<grid, 64 * WPG, lds, st>>>(t, nsb, x, xstride, nullptr, nullptr, nullptr, qmax);
  }
  return hipGetLastError();
}

template <int NR>
hipError_t launch_shape(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                        float qmax, const MvShape& sh, hipStream_t st) {
  return sh.prefetch ? launch_stream<NR, 16, true>(t, nsb, x, xstride, pre, qmax, sh.waves, st)
                     : launch_stream<NR, 16, false>(t, nsb, x, xstride, pre, qmax, sh.waves, st);
}

}  // namespace

// LDS: the activation (rows x k codes + scales + sums) and one span buffer
// per wave of a 16-wave workgroup, within a CU's 160 KiB; a row's spans must
// fit the 16 waves.
bool mv_q6k_rows_supported(int64_t k, int64_t rows) {
  return rows >= 1 && rows <= 2 && k % 256 == 0 && k >= 256 && k <= 16 * kSpanSb * 256 && k * rows <= 32768;
}

int mv_q6k_rows_per_group(int64_t k) { return 16 / (int)((k / 256 + kSpanSb - 1) / kSpanSb); }

size_t mv_q6k_rows_lds(int64_t k, int64_t rows, int wpg) {
  const int nsb = (int)(k / 256);
  return (act_lds_bytes((int)rows, nsb) + 15) / 16 * 16 + 2 * (size_t)wpg * rows * 4 + (size_t)wpg * kSpanBuf;
}

hipError_t launch_mv_q6k_rows(const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, float qmax, const MvShape& sh, hipStream_t st) {
  const int nsb = (int)(k / 256);
  if (rows == 1) return launch_shape<1>(t, nsb, x, xstride, pre, qmax, sh, st);
  return launch_shape<2>(t, nsb, x, xstride, pre, qmax, sh, st);
}

}  // namespace qmm
