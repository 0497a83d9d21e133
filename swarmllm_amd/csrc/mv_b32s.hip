// mv_b32s.hip — decode matvec (1-2 activation rows) for the 32-value block
// formats (Q8_0, IQ4_NL, MXFP4) on gfx950, streaming.
//
// Arithmetic: candle's vec_dot per type (Q8_0 k_quants.rs:1294-1312, MXFP4
// :517-527, IQ4_NL :754-764) against the activation quantized per 32 values
// (BlockQ8_0::from_float, :1240-1269), through b32_common.h: a lane's unit is
// two blocks, (dx0 dy0) s0 + (dx1 dy1) s1 with exact int32 block sums; a
// lane keeps one partial sum a row across the row's spans of 128 blocks and
// the row's sum is wave_sum_dpp of the partials: the order of the multi-row
// kernel (matvec.hip), so a row's result does not depend on the batch width.
//
// Shape of the work: each wave owns whole rows gw, gw + W, ... and walks
// their spans in order, the next span's 16-byte pieces (loaded from the
// 16-byte boundary at or before its first byte: every piece holds a byte of
// the row, and an aligned piece never crosses a page) in flight in registers
// while the current one is written to the wave's LDS buffer and computed.
// The workgroup's 16 waves fill the activation into LDS once: FUSED
// quantizes the f32 rows (8 lanes a 32-value block, the standalone
// quantizer's steps: codes and f16 scale bit-exact), else copies the
// pre-quantized planes. No barrier after the fill.
//
// One launch covers up to kMaxTargets weights of the same k sharing the
// activation (QMatMul::forward_shared): their rows are numbered one after
// another.
#include "b32_common.h"

namespace qmm {

namespace {

constexpr int kB32SpanBlocks = 128;  // 64 lanes x 2 blocks

template <int FMT>
struct B32Span {
  static constexpr int kPieces = (15 + kB32SpanBlocks * Fmt32<FMT>::B + 15) / 16;
  static constexpr int kLoads = (kPieces + 63) / 64;
  uint4 p[kLoads];
  int off;  // the span's first byte in its first piece
  int len;  // blocks in the span
};

// the activation in LDS: codes int8 [NR][k], scales f32 [NR][nb]
__host__ __device__ inline size_t b32_act_lds_bytes(int nr, int nb) {
  return (size_t)nr * nb * 32 + (size_t)nr * nb * 4;
}

template <int FMT, int NR, bool FUSED>
__global__ __launch_bounds__(1024) void mv_b32_stream_kernel(MvTargets tg, int nb, int64_t W,
                                                             const float* __restrict__ x, int64_t xstride,
                                                             const int8_t* __restrict__ yq,
                                                             const float* __restrict__ yd) {
  using F = Fmt32<FMT>;
  using Span = B32Span<FMT>;
  constexpr int kWaves = 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int k = nb * 32;
  int8_t* const acodes = (int8_t*)smem;
  float* const ad = (float*)(smem + (size_t)NR * k);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* const buf = smem + (b32_act_lds_bytes(NR, nb) + 15) / 16 * 16 + (size_t)wv * kStageBytes;
  const int64_t rowbytes = (int64_t)nb * F::B;
  const int64_t n_total = tg.row_end[tg.count - 1];
  const int nspan = (nb + kB32SpanBlocks - 1) / kB32SpanBlocks;
  const int64_t gw = (int64_t)blockIdx.x * kWaves + wv;
  const int64_t nrows = gw < n_total ? (n_total - 1 - gw) / W + 1 : 0;
  const int64_t S = nrows * nspan;  // this wave's spans

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

  // loads: span lsp of row lR
  int64_t lR = gw;
  int lsp = 0;
  const uint8_t* lrow = nullptr;
  // Past the wave's last row the loads read the first bytes of the
  // activation (cached, never used): every step issues one span's loads and
  // writes all of its pieces, so the compiler counts the loads in flight
  // exactly and waits for the oldest span only.
  const uint8_t* const idle = FUSED ? (const uint8_t*)x : (const uint8_t*)yq;
  auto load_next = [&](Span& sp) {
    const bool real = lR < n_total;
    if (lsp == 0 && real) {
      float* o;
      int64_t l;
      lrow = row_ptr(lR, o, l);
    }
    const int b0 = real ? lsp * kB32SpanBlocks : 0;
    const int len = real ? (nb - b0 < kB32SpanBlocks ? nb - b0 : kB32SpanBlocks) : 1;
    const uint8_t* p = real ? lrow + (int64_t)b0 * F::B : idle;
    sp.off = (int)((uintptr_t)p & 15);
    sp.len = len;
    const uint8_t* a0 = p - sp.off;
    const int pieces = (sp.off + len * F::B + 15) >> 4;
#pragma unroll
    for (int c = 0; c < Span::kLoads; c++) {
      const int pc = lane + 64 * c;
      sp.p[c] = ld_stream16(a0 + 16u * (uint32_t)(pc < pieces ? pc : pieces - 1));
    }
    if (++lsp == nspan) {
      lsp = 0;
      lR += W;
    }
  };

  // 1. the activation's loads (FUSED: 4 values a thread, 8 threads a block), then the first spans'
  const int nblk = NR * nb;
  constexpr int kPre = 2;  // passes of 1024 threads loaded before the weights
  float4 xv[kPre];
  int8_t* dummy = nullptr;
  (void)dummy;
  auto xload = [&](int pass) -> float4 {
    const int t = pass * 1024 + (int)threadIdx.x;
    const int blk = t >> 3, sub = t & 7;
    if (blk >= nblk) return make_float4(0.f, 0.f, 0.f, 0.f);
    const int r = blk / nb, b = blk - r * nb;
    return *(const float4*)(x + r * xstride + b * 32 + 4 * sub);  // rows 16-byte aligned (the launcher checks)
  };
  if (FUSED) {
#pragma unroll
    for (int p = 0; p < kPre; p++) xv[p] = xload(p);
  }
  Span sa, sb;
  load_next(sa);
  load_next(sb);

  // 2. the activation into LDS
  auto quant_pass = [&](int pass, const float4& v4) {
#pragma clang fp contract(off)
    const int t = pass * 1024 + (int)threadIdx.x;
    const int blk = t >> 3, sub = t & 7;
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    // amax as f32::max folds it (fmaxf ignores NaN the same way); >= 0, so
    // the 8-lane maximum (DPP within rows of 16) is taken on its bits
    const float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    uint32_t ab = __float_as_uint(fmaxf(am, 0.0f));
    ab = max(ab, dpp_u<0xB1>(ab));
    ab = max(ab, dpp_u<0x4E>(ab));
    ab = max(ab, dpp_u<0x141>(ab));
    const float amax = __uint_as_float(ab);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint32_t packed = pack4_i8(q8_0_code(v[0] * id), q8_0_code(v[1] * id), q8_0_code(v[2] * id), q8_0_code(v[3] * id));
    if (blk < nblk) {
      const int r = blk / nb, b = blk - r * nb;
      *(uint32_t*)(acodes + r * k + b * 32 + 4 * sub) = packed;
      if (sub == 0) ad[r * nb + b] = h2f(f2h(d));
    }
  };
  if (FUSED) {
#pragma unroll
    for (int p = 0; p < kPre; p++) quant_pass(p, xv[p]);
    for (int p = kPre; p * 128 < nblk; p++) quant_pass(p, xload(p));
  } else {
    for (int i = (int)threadIdx.x; i < NR * k / 16; i += 1024) {
      const int r = (i * 16) / k, o = i * 16 - r * k;
      *(uint4*)(acodes + r * k + o) = *(const uint4*)(yq + (int64_t)r * k + o);
    }
    for (int i = (int)threadIdx.x; i < nblk; i += 1024) ad[i] = yd[i];
  }
  __syncthreads();

  // 3. the spans, in order: stage, reload the buffer with the span two ahead, compute
  const Lut32<FMT> lut;
  const uint32_t t0 = lut.t0, t1 = lut.t1, t2 = lut.t2, t3 = lut.t3;
  const int bl = 2 * lane;  // the lane's unit: blocks bl, bl+1 of the span
  int64_t R = gw;
  int sp = 0;
  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) acc[r] = 0.0f;

  auto step = [&](Span& cur, int64_t sigma) {
    wave_lds_sync();
#pragma unroll
    for (int c = 0; c < Span::kLoads; c++) {
      const int pc = lane + 64 * c;
      *(uint4*)(buf + 16 * (pc < Span::kPieces ? pc : Span::kPieces - 1)) = cur.p[c];
    }
    wave_lds_sync();
    const int off = cur.off, len = cur.len;
    load_next(cur);
    if (sigma >= S) return;
    if (bl < len) {
      const bool two = bl + 1 < len;
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
      const int gb = sp * kB32SpanBlocks + bl;
#pragma unroll
      for (int r = 0; r < NR; r++) {
        Act64 a;
        const int4* yp = (const int4*)(acodes + r * k + gb * 32);
        const int4 a0 = yp[0], a1 = yp[1];
        a.y[0][0] = a0.x; a.y[0][1] = a0.y; a.y[0][2] = a0.z; a.y[0][3] = a0.w;
        a.y[0][4] = a1.x; a.y[0][5] = a1.y; a.y[0][6] = a1.z; a.y[0][7] = a1.w;
        a.dy[0] = ad[r * nb + gb];
        if (two) {
          const int4 b0 = yp[2], b1 = yp[3];
          a.y[1][0] = b0.x; a.y[1][1] = b0.y; a.y[1][2] = b0.z; a.y[1][3] = b0.w;
          a.y[1][4] = b1.x; a.y[1][5] = b1.y; a.y[1][6] = b1.z; a.y[1][7] = b1.w;
          a.dy[1] = ad[r * nb + gb + 1];
        } else {
#pragma unroll
          for (int t = 0; t < 8; t++) a.y[1][t] = 0;
          a.dy[1] = 0.0f;
        }
        acc[r] = b32_unit(q0, q1, dx0, dx1, a, acc[r]);
      }
    }
    if (++sp == nspan) {
      float* out;
      int64_t ldd;
      (void)row_ptr(R, out, ldd);
#pragma unroll
      for (int r = 0; r < NR; r++) {
        const float v = wave_sum_dpp(acc[r]);
        if (lane == 0) out[r * ldd] = v;
        acc[r] = 0.0f;
      }
      sp = 0;
      R += W;
    }
  };
  for (int64_t sigma = 0; sigma < S; sigma += 2) {
    step(sa, sigma);
    step(sb, sigma + 1);
  }
}

template <int FMT, int NR>
hipError_t launch_b32s(const MvTargets& t, int nb, const float* x, int64_t xstride, const ActPlanes* pre, int cus,
                       hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t n_total = t.row_end[t.count - 1];
  int64_t waves = (int64_t)cus * 16;
  // every wave the same number of rows (the last ones one fewer)
  const int64_t rpw = (n_total + waves - 1) / waves;
  waves = (n_total + rpw - 1) / rpw;
  waves = (waves + 15) / 16 * 16;
  const size_t lds = (b32_act_lds_bytes(NR, nb) + 15) / 16 * 16 + 16 * (size_t)kStageBytes;
  const dim3 grid((unsigned)(waves / 16));
  if (pre) {
    constexpr auto* kfn = &mv_b32_stream_kernel<FMT, NR, false>;
    if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
    kfn<<<grid, 1024, lds, st>>>(t, nb, waves, nullptr, 0, pre->codes, pre->d);
  } else {
    constexpr auto* kfn = &mv_b32_stream_kernel<FMT, NR, true>;
    if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
    kfn<<<grid, 1024, lds, st>>>(t, nb, waves, x, xstride, nullptr, nullptr);
  }
  return hipGetLastError();
}

template <int NR>
hipError_t launch_b32s_nr(int type, const MvTargets& t, int nb, const float* x, int64_t xstride,
                          const ActPlanes* pre, int cus, hipStream_t st) {
  switch (type) {
    case T_Q8_0: return launch_b32s<T_Q8_0, NR>(t, nb, x, xstride, pre, cus, st);
    case T_IQ4_NL: return launch_b32s<T_IQ4_NL, NR>(t, nb, x, xstride, pre, cus, st);
    case T_MXFP4: return launch_b32s<T_MXFP4, NR>(t, nb, x, xstride, pre, cus, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// LDS: the activation and one stage buffer per wave of a 16-wave workgroup,
// within a CU's 160 KiB.
bool mv_b32_rows_supported(int type, int64_t k, int64_t rows) {
  if (type != T_Q8_0 && type != T_IQ4_NL && type != T_MXFP4) return false;
  if (rows < 1 || rows > 2 || k % 32 != 0 || k < 32) return false;
  return (b32_act_lds_bytes((int)rows, (int)(k / 32)) + 15) / 16 * 16 + 16 * (size_t)kStageBytes <= 160 * 1024;
}

hipError_t launch_mv_b32_rows(int type, const MvTargets& t, int64_t k, int64_t rows, const float* x, int64_t xstride,
                              const ActPlanes* pre, int cus, hipStream_t st) {
  const int nb = (int)(k / 32);
  if (rows == 1) return launch_b32s_nr<1>(type, t, nb, x, xstride, pre, cus, st);
  return launch_b32s_nr<2>(type, t, nb, x, xstride, pre, cus, st);
}

}  // namespace qmm
