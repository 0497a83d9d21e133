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

// Work: each wave owns whole rows, gw, gw + W, ... (gw its index among the
// W waves of the grid), and walks their spans in order with the loads of the
// next kPfd spans in flight in a register ring (the loop is unrolled by kPfd,
// so every buffer keeps its registers). A span is written to the wave's LDS
// buffer, read back per lane, reduced (wave_sum_dpp) and added to its row's
// sum in span order: the arithmetic of the multi-row kernel (matvec.hip), so
// a row's result does not depend on the batch width. No barrier after the
// activation fill: the waves run independently.
//
// Every step issues exactly one span's loads and writes all of its pieces,
// whatever the position in the wave's work: past the wave's last span the
// loads read a cached piece of the activation (never used) and lanes past a
// span's pieces write their copy of its last piece to the slack piece. Only
// the arithmetic and the output store depend on the position. The compiler
// then counts the loads in flight exactly and waits for the oldest span only;
// a load issued on one path and not another would make it wait for them all.
//
// Spans in flight per wave: one, the next span's loads issued while the
// current one is computed. Measured on C2's down projection (4096 x 14336,
// a row per wave): 14.6 us with one span in flight, 16.1 us with two, 18.0 us
// with three; more requests outstanding at once (41 MB with three) lower
// what HBM delivers rather than hide more latency. Measured again with every
// step's loads unconditional (exact wait counts): the C2 layer step takes
// 36.7-37.1 us with one span in flight, 38.2-38.3 us with two.
constexpr int kPfd = 1;

template <int NR, bool FUSED>
__global__ __launch_bounds__(1024) void mv_q6k_stream_kernel(MvTargets tg, int nsb, int W,
                                                             const float* __restrict__ x, int64_t xstride,
                                                             const int8_t* __restrict__ yq,
                                                             const float* __restrict__ yd,
                                                             const int16_t* __restrict__ ybs, float qmax) {
  constexpr int kWaves = 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const ActLds s = act_lds(smem, NR, nsb);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + (act_lds_bytes(NR, nsb) + 15) / 16 * 16 + (size_t)wv * kQ6SpanBuf;
  const int k = nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 210;
  // row numbers fit an int (the host checks)
  const int n_total = (int)tg.row_end[tg.count - 1];
  const int nspan = (nsb + kQ6SpanSb - 1) / kQ6SpanSb;
  const int gw = blockIdx.x * kWaves + wv;
  // spans of this wave: its rows times the spans of a row
  const int nrows = gw < n_total ? (n_total - 1 - gw) / W + 1 : 0;
  const int S = nrows * nspan;

  auto target_of = [&](int R, int& lrow) {
    int t = 0;
#pragma unroll
    for (int q = 0; q < kMaxTargets - 1; q++)
      if (q < tg.count - 1 && R >= (int)tg.row_end[q]) t = q + 1;
    lrow = R - (t ? (int)tg.row_end[t - 1] : 0);
    return t;
  };

  // the loads: span lsp of row lR, whose bytes start at lrow; past the
  // wave's last row, the first 224 bytes of the activation (16-byte aligned,
  // at least 256 bytes long, and just read by every workgroup, so cached)
  int lR = gw, lsp = 0;
  const uint8_t* lrow = nullptr;
  const uint8_t* const idle = FUSED ? (const uint8_t*)x : (const uint8_t*)yq;
  auto load_next = [&](Q6Span& sp) {
    if (lsp == 0 && lR < n_total) {
      int lr;
      const int t = target_of(lR, lr);
      lrow = (const uint8_t*)tg.w[t] + (int64_t)lr * rowbytes;
    }
    const int s0 = lsp * kQ6SpanSb;
    if (lR < n_total)
      load_q6_span(sp, lrow + (int64_t)s0 * 210, nsb - s0 < kQ6SpanSb ? nsb - s0 : kQ6SpanSb, lane);
    else
      load_q6_span(sp, idle, 1, lane);
    if (++lsp == nspan) {
      lsp = 0;
      lR += W;
    }
  };

  // 1. activation loads, then the first spans' loads
  ActBatch<NR, FUSED, kWaves> act;
  act.load(nsb, x, xstride, yq, yd, ybs);
  Q6Span ring[kPfd];
#pragma unroll
  for (int j = 0; j < kPfd; j++) load_next(ring[j]);

  // 2. the activation into LDS
  act.store(s, nsb, x, xstride, yq, yd, ybs, qmax);
  __syncthreads();

  // 3. the spans, in order
  const int sbl = lane >> 2, u = lane & 3, h = u >> 1, l0 = 16 * (u & 1);
  int R = gw;  // the span being computed: span sp of row R
  int sp = 0;
  float tot[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) tot[r] = 0.0f;

  auto step = [&](Q6Span& cur, int sigma) {
    // the span into this wave's LDS buffer (the previous span's reads are done)
    wave_lds_sync();
#pragma unroll
    for (int c = 0; c < kQ6PiecesPerLane; c++) {
      const int pc = lane + 64 * c;
      *(uint4*)(buf + 16 * (pc < kQ6SpanPieces ? pc : kQ6SpanPieces - 1)) = cur.p[c];
    }
    wave_lds_sync();
    const int off = cur.off, len = cur.len;
    // this buffer's next span
    load_next(cur);
    if (sigma >= S) return;
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.0f;
    if (sbl < len) {
      Q6Lane u;
      load_q6_lane(buf, off + 210 * sbl, h, l0, u);
      const int sb = sp * kQ6SpanSb + sbl;
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
        acc[r] = q6k_unit(u.qlA, u.qlB, u.qh, u.sc, u.dx, yv, s.dy[r * nsb + sb], bs, acc[r]);
      }
    }
    // the span's sum, added to its row's in span order
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const float v = wave_sum_dpp(acc[r]);
      tot[r] = sp == 0 ? v : __fadd_rn(tot[r], v);
    }
    if (++sp == nspan) {
      if (lane == 0) {
        int lr;
        const int t = target_of(R, lr);
        float* out = tg.dst[t] + lr;
#pragma unroll
        for (int r = 0; r < NR; r++) out[r * tg.ldd[t]] = tot[r];
      }
      sp = 0;
      R += W;
    }
  };

  for (int sigma = 0; sigma < S; sigma += kPfd) {
#pragma unroll
    for (int j = 0; j < kPfd; j++) step(ring[j], sigma + j);
  }
}

// one workgroup of 16 waves a CU (up to 128 registers a lane), a wave a row
// where the rows are few
template <int NR>
hipError_t launch_stream(const MvTargets& t, int nsb, const float* x, int64_t xstride, const ActPlanes* pre,
                         float qmax, int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t n_total = t.row_end[t.count - 1];
  if (n_total >= ((int64_t)1 << 30)) return hipErrorInvalidValue;  // row numbers are ints in the kernel
  int waves = cus * 16;
  if (waves > n_total) waves = (int)((n_total + 15) / 16 * 16);
  const size_t lds = (act_lds_bytes(NR, nsb) + 15) / 16 * 16 + 16 * (size_t)kQ6SpanBuf;
  const dim3 grid((unsigned)(waves / 16));
  if (pre) {
    constexpr auto* kfn = &mv_q6k_stream_kernel<NR, false>;
    if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
    kfn<<<grid, 1024, lds, st>>>(t, nsb, waves, nullptr, 0, pre->codes, pre->d, (const int16_t*)pre->sums, qmax);
  } else {
    constexpr auto* kfn = &mv_q6k_stream_kernel<NR, true>;
    if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
    kfn<<<grid, 1024, lds, st>>>(t, nsb, waves, x, xstride, nullptr, nullptr, nullptr, qmax);
  }
  return hipGetLastError();
}

}  // namespace

// LDS: the activation (rows x k codes + scales + sums) and one span buffer
// per wave of a 16-wave workgroup, within a CU's 160 KiB.
bool mv_q6k_rows_supported(int64_t k, int64_t rows) {
  return rows >= 1 && rows <= 2 && k % 256 == 0 && k >= 256 && k * rows <= 65536;
}

hipError_t launch_mv_q6k_rows(const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, float qmax, int cus, hipStream_t st) {
  const int nsb = (int)(k / 256);
  if (rows == 1) return launch_stream<1>(t, nsb, x, xstride, pre, qmax, cus, st);
  return launch_stream<2>(t, nsb, x, xstride, pre, qmax, cus, st);
}

}  // namespace qmm
