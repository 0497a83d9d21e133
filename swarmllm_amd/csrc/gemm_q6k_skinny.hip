// gemm_q6k_skinny.hip — Q6_K products of a few activation rows (4 to 32) on
// the int8 matrix cores of gfx950.
//
// The arithmetic is candle's Q6_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2598-2655) with the
// inner sums as matrix-core products. Per super-block and 16-value group j
// (scale sc_j, int8) the exact int32
//   C_j = sum_{16} q y          q the unsigned 6-bit code (ql nibble | qh << 4)
//   S   = sum_j sc_j sum_{16} y (the activation's group sums against the scales)
// give tot = sum_j sc_j C_j - 32 S = sum_j sc_j sum (q - 32) y, the
// reference's integer sum, and acc += (d dy) tot in f32.
//
// Shape: v_mfma_i32_16x16x64_i8 with the activation rows on the A side (MT
// tiles of 16) and 16 weight rows on the B side. A 64-deep K-chunk c holds
// the groups 4c .. 4c+3, one per 16-lane group of the wave (lane L: weight
// row L%16, group 4c + L/16, its 16 values). A group's scale differs per
// weight row, so each chunk runs four products, the activation fragment
// masked to one lane group in each, and scales their int32 results on the
// vector unit; one more product with the scales broadcast over their groups
// gives S. A workgroup owns NB tiles of 16 weight rows; its kWaves waves
// split the super-blocks of K and add their partial sums through LDS in
// wave order. A wave streams its super-blocks: per row the 14 16-byte
// pieces from the boundary at or before the block's first byte (every piece
// holds a byte of the block, and an aligned piece never crosses a page), the
// next two super-blocks in flight in registers, written to the wave's LDS
// buffer and read back with dword reads and alignbyte. It takes the products
// the reference sends to its int8 MMQ from 4 rows on weights of 2 MiB or more
// (mmq_takes_few_rows, quantized/cuda.rs:790-839).
//
// One launch covers up to kMaxTargets weights sharing the activation: their
// rows are numbered one after another. Rows past a target's end, and
// activation rows past M, are read clamped and never stored.
#include "mv_common.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// two 16-bit multiply-adds in one instruction (v_pk_mad_u16)
__device__ __forceinline__ uint32_t pkmad16(uint32_t a, uint32_t b, uint32_t c) {
  const u16x2 x = __builtin_bit_cast(u16x2, a), y = __builtin_bit_cast(u16x2, b), z = __builtin_bit_cast(u16x2, c);
  return __builtin_bit_cast(uint32_t, x * y + z);
}
// ONE: the weight as w8 = round(m_j (q - 32) / 256) with m_j = round(127
// sc_j / 16), so sc_j (q - 32) ~ (4096 / 127) w8 (the single-pass GEMM's
// form, gemm_q4k_sp.hip): one product a 64-deep chunk instead of five
constexpr float kQ6One = 4096.0f / 127.0f;

constexpr int kQ6Win = 224;  // bytes staged a row: 14 pieces cover the 210-byte block at any offset
// LDS bytes between staged rows: 57 dwords, so the same dword of the 16 rows
// a read spans falls on 16 different banks (at 224 bytes, 56 dwords, the 16
// rows share 4 of them and each of the block's dword reads waited 4 times as
// long). The pieces are then only 4-byte aligned and go in as dwords.
constexpr int kQ6Row = kQ6Win + 4;

template <int NB>
struct Q6Pieces {
  static constexpr int P = 16 * NB * 14;
  static constexpr int L = (P + 63) / 64;
  uint4 v[L];
};

template <int MT>
struct Q6Act {
  i4v a[MT][4];
  float dy[MT][4];
};

template <int MT, int NB, int kWaves, bool ONE>
__global__ __launch_bounds__(64 * kWaves) void gemm_q6k_skinny_kernel(MvTargets tg, int nsb,
                                                                      const int8_t* __restrict__ yq,
                                                                      const float* __restrict__ yd, int M) {
  constexpr int ROWS = 16 * NB;
  using Pieces = Q6Pieces<NB>;
  constexpr int L = Pieces::L;
  constexpr int kBuf = ROWS * kQ6Row + 16 > NB * MT * 4 * 64 * 4 ? ROWS * kQ6Row + 16 : NB * MT * 4 * 64 * 4;
  __shared__ __attribute__((aligned(16))) uint8_t sbuf[kWaves][kBuf];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int64_t K = (int64_t)nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 210;
  const int64_t n_total = tg.row_end[tg.count - 1];
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  uint8_t* const buf = sbuf[wv];

  const int per = (nsb + kWaves - 1) / kWaves;
  const int sb0 = wv * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;

  auto row_ptr = [&](int64_t R, int& t, int64_t& lrow) -> const uint8_t* {
    R = R < n_total ? R : n_total - 1;
    t = 0;
#pragma unroll
    for (int i = 0; i < kMaxTargets - 1; i++)
      if (i < tg.count - 1 && R >= tg.row_end[i]) t = i + 1;
    lrow = R - (t ? tg.row_end[t - 1] : 0);
    return (const uint8_t*)tg.w[t] + lrow * rowbytes;
  };

  // the lane's pieces: piece p = lane + 64 t is piece p % 14 of row p / 14
  const uint8_t* prow[L];
  int pj[L];
#pragma unroll
  for (int t = 0; t < L; t++) {
    const int p = lane + 64 * t;
    const int pp = p < Pieces::P ? p : Pieces::P - 1;
    int tt;
    int64_t lr;
    prow[t] = row_ptr(row0 + pp / 14, tt, lr);
    pj[t] = pp % 14;
  }
  auto load_w = [&](Pieces& pc, int sb) {
#pragma unroll
    for (int t = 0; t < L; t++) {
      const uint8_t* s = prow[t] + (int64_t)sb * 210;
      pc.v[t] = ld_stream16(s - ((uintptr_t)s & 15) + 16 * pj[t]);
    }
  };
  // every lane writes (lanes past the pieces rewrite the last piece, which
  // they loaded too): no branch, so the loads' wait counts stay exact
  auto stage_w = [&](const Pieces& pc) {
#pragma unroll
    for (int t = 0; t < L; t++) {
      const int p = lane + 64 * t;
      const int pp = p < Pieces::P ? p : Pieces::P - 1;
      uint32_t* const d = (uint32_t*)(buf + (pp / 14) * kQ6Row + 16 * (pp % 14));
      d[0] = pc.v[t].x;
      d[1] = pc.v[t].y;
      d[2] = pc.v[t].z;
      d[3] = pc.v[t].w;
    }
  };
  // the block offset of the lane's own rows within their staged windows
  int rlo[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) {
    int tt;
    int64_t lr;
    rlo[b] = (int)((uintptr_t)row_ptr(row0 + 16 * b + r16, tt, lr) & 15);
  }

  int64_t arow[MT];
  int64_t crow[MT][4];
#pragma unroll
  for (int m = 0; m < MT; m++) {
    arow[m] = 16 * m + r16 < M ? 16 * m + r16 : M - 1;
#pragma unroll
    for (int i = 0; i < 4; i++) crow[m][i] = 16 * m + 4 * kq + i < M ? 16 * m + 4 * kq + i : M - 1;
  }
  auto load_a = [&](Q6Act<MT>& r, int sb) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
      for (int c = 0; c < 4; c++) r.a[m][c] = *(const i4v*)(yq + arow[m] * K + (int64_t)sb * 256 + 64 * c + 16 * kq);
#pragma unroll
      for (int i = 0; i < 4; i++) r.dy[m][i] = yd[crow[m][i] * nsb + sb];
    }
  };

  float acc[NB][MT][4];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[b][m][i] = 0.0f;

  // lane group masks: the activation fragment of group g only
  uint32_t gmask[4];
#pragma unroll
  for (int g = 0; g < 4; g++) gmask[g] = kq == g ? 0xFFFFFFFFu : 0u;

  auto compute = [&](const Q6Act<MT>& act, int sb) {
    // each f32 operation rounded on its own (no contraction into fma)
#pragma clang fp contract(off)
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const uint8_t* rowp = buf + (16 * b + r16) * kQ6Row;
      const int o = (rlo[b] + 210 * sb) & 15;
      uint32_t ql[2][4], qh[2][4], scw[4];
      lds_words<4>(rowp, o + 16 * kq, ql[0]);
      lds_words<4>(rowp, o + 64 + 16 * kq, ql[1]);
      lds_words<4>(rowp, o + 128 + 16 * (kq & 1), qh[0]);
      lds_words<4>(rowp, o + 160 + 16 * (kq & 1), qh[1]);
      lds_words<4>(rowp, o + 192, scw);
      const float dw = h2f((uint16_t)lds_u16(rowp, o + 208));

      const i4v zero = {0, 0, 0, 0};
      if constexpr (ONE) {
        i4v T[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) T[m] = zero;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int hh = c >> 1, nib = 4 * (c & 1);
          const int qsh = 4 * (c & 1) + 2 * (kq >> 1);
          // this lane's group 4c + L/16 of its weight row: multiplier m and
          // per 16-bit lane m (q - 32) + 128, whose high byte is w8
          const int sc = (int)(int8_t)((scw[c] >> (8 * kq)) & 0xFF);
          const int mj = (127 * sc + 8) >> 4;
          const uint32_t Mw = ((uint32_t)mj & 0xFFFFu) * 0x10001u, Cw = ((uint32_t)(128 - 32 * mj) & 0xFFFFu) * 0x10001u;
          i4v w8;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t q = ((ql[hh][e] >> nib) & 0x0F0F0F0Fu) | (((qh[hh][e] >> qsh) & 0x03030303u) << 4);
            const uint32_t ev = pkmad16(q & 0x00FF00FFu, Mw, Cw), od = pkmad16((q >> 8) & 0x00FF00FFu, Mw, Cw);
            w8[e] = (int)__builtin_amdgcn_perm(od, ev, 0x07030501u);
          }
#pragma unroll
          for (int m = 0; m < MT; m++) T[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(act.a[m][c], w8, T[m], 0, 0, 0);
        }
        // |T| <= 256 * 127 * 127 < 2^24: exact in f32
        const float dq = dw * kQ6One;
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[b][m][i] = acc[b][m][i] + (dq * act.dy[m][i]) * (float)T[m][i];
        continue;
      }
      i4v tot[MT], S[MT];
#pragma unroll
      for (int m = 0; m < MT; m++) tot[m] = zero;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int hh = c >> 1, nib = 4 * (c & 1);
        const int qsh = 4 * (c & 1) + 2 * (kq >> 1);  // this lane's group: qd = 2 (c%2) + L/32
        i4v bq;
#pragma unroll
        for (int e = 0; e < 4; e++)
          bq[e] = (int)(((ql[hh][e] >> nib) & 0x0F0F0F0Fu) | (((qh[hh][e] >> qsh) & 0x03030303u) << 4));
        // the scales of groups 4c .. 4c+3 of this lane's weight row (the C column)
        const uint32_t sw = scw[c];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int sc = (int)(int8_t)((sw >> (8 * g)) & 0xFF);
#pragma unroll
          for (int m = 0; m < MT; m++) {
            i4v ag;
#pragma unroll
            for (int e = 0; e < 4; e++) ag[e] = (int)((uint32_t)act.a[m][c][e] & gmask[g]);
            const i4v cg = __builtin_amdgcn_mfma_i32_16x16x64_i8(ag, bq, zero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) tot[m][i] += __mul24(sc, cg[i]);  // |cg| < 2^17
          }
        }
        // S: this lane's group's scale over its 16 values
        const int sl = (int)(((sw >> (8 * kq)) & 0xFF) * 0x01010101u);
        const i4v bs = {sl, sl, sl, sl};
#pragma unroll
        for (int m = 0; m < MT; m++) S[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(act.a[m][c], bs, c == 0 ? zero : S[m], 0, 0, 0);
      }
#pragma unroll
      for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = tot[m][i] - 32 * S[m][i];
          acc[b][m][i] = acc[b][m][i] + (dw * act.dy[m][i]) * (float)t;
        }
    }
  };

  // A step stages super-block sb, issues the weight loads of sb + 2,
  // computes sb and then reloads the activation registers it just used with
  // sb + 2: a wave's loads complete in issue order, so an activation load
  // issued ahead of the compute would make the next compute wait for the
  // weights issued before it (see gemm_q4k_skinny.hip). The main loop runs
  // while both of its steps have all their loads, which it then issues
  // unconditionally (a load issued on one path and not another makes the
  // compiler wait for every load in flight); the last steps follow it,
  // loading only what remains.
  Pieces pa, pb;
  Q6Act<MT> aa, ab;
  if (sb0 < sb1) {
    load_w(pa, sb0);
    load_a(aa, sb0);
    if (sb0 + 1 < sb1) {
      load_w(pb, sb0 + 1);
      load_a(ab, sb0 + 1);
    }
  }
  // the matrix work at a raised wave priority, as in gemm_q4k_skinny.hip
  auto step_full = [&](Pieces& pc, Q6Act<MT>& cur, int sb) {
    wave_lds_sync();
    stage_w(pc);
    load_w(pc, sb + 2);
    wave_lds_sync();
    __builtin_amdgcn_s_setprio(1);
    compute(cur, sb);
    __builtin_amdgcn_s_setprio(0);
    load_a(cur, sb + 2);
  };
  auto step_tail = [&](Pieces& pc, Q6Act<MT>& cur, int sb) {
    wave_lds_sync();
    stage_w(pc);
    if (sb + 2 < sb1) load_w(pc, sb + 2);
    wave_lds_sync();
    compute(cur, sb);
    if (sb + 2 < sb1) load_a(cur, sb + 2);
  };
  int sb = sb0;
  for (; sb + 3 < sb1; sb += 2) {
    step_full(pa, aa, sb);
    step_full(pb, ab, sb + 1);
  }
  if (sb < sb1) step_tail(pa, aa, sb);
  if (sb + 1 < sb1) step_tail(pb, ab, sb + 1);
  if (sb + 2 < sb1) step_tail(pa, aa, sb + 2);

  wave_lds_sync();
  float* part = (float*)buf;
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) part[((b * MT + m) * 4 + i) * 64 + lane] = acc[b][m][i];
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int64_t R = row0 + 16 * b + r16;
      if (R >= n_total) continue;
      int t;
      int64_t lrow;
      (void)row_ptr(R, t, lrow);
      float* out = tg.dst[t] + lrow;
      const int64_t ldd = tg.ldd[t];
#pragma unroll
      for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int idx = ((b * MT + m) * 4 + i) * 64 + lane;
          float v = ((const float*)sbuf[0])[idx];
#pragma unroll
          for (int w = 1; w < kWaves; w++) v = __fadd_rn(v, ((const float*)sbuf[w])[idx]);
          const int ar = 16 * m + 4 * kq + i;
          if (ar < M) out[(int64_t)ar * ldd] = v;
        }
    }
  }
}

template <int MT, int NB, int W, bool ONE>
hipError_t launch_q6(const MvTargets& t, int nsb, const ActPlanes& p, int64_t rows, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t n_total = t.row_end[t.count - 1];
  const dim3 grid((unsigned)((n_total + 16 * NB - 1) / (16 * NB)));
  gemm_q6k_skinny_kernel<MT, NB, W, ONE><<<grid, 64 * W, 0, st>>>(t, nsb, p.codes, p.d, (int)rows);
  return hipGetLastError();
}

}  // namespace

bool gemm_q6k_skinny_fits(int64_t k, int64_t rows) { return k % 256 == 0 && rows >= 1 && rows <= 32; }

hipError_t launch_gemm_q6k_skinny(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, int cus,
                                  hipStream_t st) {
  (void)cus;
  const int nsb = (int)(k / 256);
  // the single-product form from k = 2048 (its rounding stays well inside
  // the 2e-3 bound there); shorter rows, and every row under
  // SWARMLLM_QMATMUL_EXACT, keep the exact form
  if (k >= 2048 && !exact_forms()) {
    if (rows <= 16) return launch_q6<1, 1, 4, true>(t, nsb, p, rows, st);
    return launch_q6<2, 1, 4, true>(t, nsb, p, rows, st);
  }
  if (rows <= 16) return launch_q6<1, 1, 4, false>(t, nsb, p, rows, st);
  return launch_q6<2, 1, 4, false>(t, nsb, p, rows, st);
}

}  // namespace qmm
