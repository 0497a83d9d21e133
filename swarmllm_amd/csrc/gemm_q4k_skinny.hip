// gemm_q4k_skinny.hip — Q4_K products of a few activation rows (speculative
// verification widths: 4 to 32) on the int8 matrix cores of gfx950.
//
// The arithmetic is the prefill GEMM's (gemm_q4k.hip): per super-block the
// exact int32 T = sum_j sc_j sum q y from two int8 MFMA passes over the weight
// with its 6-bit scale split sc = 8 sh + sl (sh q and sl q fit int8), then
// acc += (dy_m d_n) T in f32 and the min term f16(dy_m S_mj) x
// f16(-dmin_n m_nj) as an f16 MFMA — candle's Q4_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2031-2111). It takes
// the products the reference sends to its int8 MMQ from 4 rows on weights of
// 2 MiB or more (mmq_takes_few_rows, quantized/cuda.rs:790-839).
//
// Shape: v_mfma_i32_16x16x64_i8 with the activation rows on the A side (M
// padded to 16 or 32 rows: MT tiles of 16) and 16 weight rows on the B side.
// A workgroup takes 16-row weight tiles gridDim.x apart (the launch gives
// each its own); its kWaves waves split the super-blocks of K
// between them and add their partial sums of a tile through LDS in wave
// order (deterministic). Each wave keeps the raw weight bytes of the
// next two super-blocks in flight while it multiplies the current one. Lane L of a
// wave holds weight row L%16 and, of each 64-deep K-chunk c, the 16 code
// bytes 32c + 16((L/16)%2): its B-operand bytes (low nibbles for L/16 < 2,
// high nibbles otherwise). Activation fragments and scales come straight
// from the quantized planes (cache-resident: every workgroup reads the same
// rows), one super-block ahead like the weights.
//
// One launch covers up to kMaxTargets weights sharing the activation (q/k/v,
// gate/up): their rows are numbered one after another. Rows past a target's
// end, and activation rows past M, are read clamped and never stored.
#include "mv_common.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kSkWaves = 4;

__device__ __forceinline__ uint32_t sk_dup16(uint32_t v) { return v | (v << 16); }

__device__ __forceinline__ uint32_t sk_pkmul(uint32_t a, uint32_t s2) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, s2);
  return __builtin_bit_cast(uint32_t, x * y);
}

__device__ __forceinline__ uint32_t sk_word(const uint4& c, int e) {
  return e == 0 ? c.x : e == 1 ? c.y : e == 2 ? c.z : c.w;
}

// The raw bytes a lane reads of its weight row for one super-block.
struct SkRaw {
  uint4 hdr;             // d, dmin, 12 scale bytes
  uint4 c0, c1, c2, c3;  // code bytes 32c + 16 ((L/16) % 2) .. +15, c = 0..3
};

__device__ __forceinline__ const uint4& sk_chunk(const SkRaw& r, int c) {
  return c == 0 ? r.c0 : c == 1 ? r.c1 : c == 2 ? r.c2 : r.c3;
}

template <int MT>
__global__ __launch_bounds__(64 * kSkWaves) void gemm_q4k_skinny_kernel(MvTargets tg, int nsb,
                                                                        const int8_t* __restrict__ yq,
                                                                        const float* __restrict__ yd,
                                                                        const int16_t* __restrict__ ybs, int M) {
  __shared__ float part[kSkWaves][MT][4][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int64_t K = (int64_t)nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;
  const int64_t n_total = tg.row_end[tg.count - 1];

  const int64_t ntiles = (n_total + 15) / 16;
  const int hb = 16 * (kq & 1);  // byte offset of this lane's 16 code bytes within a 32-byte chunk
  const bool hin = kq >= 2;      // this lane's K-slices are high nibbles

  // the super-blocks of this wave (the same for every tile)
  const int per = (nsb + kSkWaves - 1) / kSkWaves;
  const int sb0 = wv * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  const bool work = sb0 < sb1;

  // activation rows of this lane's A fragments (clamped to M - 1)
  int64_t arow[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) arow[m] = 16 * m + r16 < M ? 16 * m + r16 : M - 1;

  // this lane's weight row of a tile: target, row within it (clamped to the last row)
  auto tile_row = [&](int64_t tile, int& t, int64_t& lrow) -> const uint8_t* {
    const int64_t R = tile * 16 + r16 < n_total ? tile * 16 + r16 : n_total - 1;
    t = 0;
#pragma unroll
    for (int i = 0; i < kMaxTargets - 1; i++)
      if (i < tg.count - 1 && R >= tg.row_end[i]) t = i + 1;
    lrow = R - (t ? tg.row_end[t - 1] : 0);
    return (const uint8_t*)tg.w[t] + lrow * rowbytes;
  };
  auto load_w = [&](SkRaw& r, int64_t tile, int sb) {
    int tt;
    int64_t lr;
    const uint8_t* blk = tile_row(tile, tt, lr) + (int64_t)sb * 144;
    r.hdr = ld_stream16(blk);
    r.c0 = *(const uint4*)(blk + 16 + hb);
    r.c1 = *(const uint4*)(blk + 48 + hb);
    r.c2 = *(const uint4*)(blk + 80 + hb);
    r.c3 = *(const uint4*)(blk + 112 + hb);
  };

  // The activation of a super-block: A fragments (chunk c, lane k-slice
  // 16 kq), the scales of the epilogue's rows 16m + 4kq + i, and (lanes
  // kq == 0) the min term's f16(dy S_j) of row arow[m].
  struct SkAct {
    i4v a[MT][4];
    float dy[MT][4];
    float dya[MT];      // scale of row arow[m] (min term)
    uint4 bs[MT][2];    // its 16 group sums
  };
  auto load_act = [&](SkAct& r, int sb) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
      for (int c = 0; c < 4; c++) r.a[m][c] = *(const i4v*)(yq + arow[m] * K + (int64_t)sb * 256 + 64 * c + 16 * kq);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int ar = 16 * m + 4 * kq + i < M ? 16 * m + 4 * kq + i : M - 1;
        r.dy[m][i] = yd[(int64_t)ar * nsb + sb];
      }
      r.dya[m] = yd[arow[m] * nsb + sb];
      const int16_t* bs = ybs + arow[m] * (K / 16) + (int64_t)sb * 16;
      r.bs[m][0] = *(const uint4*)bs;
      r.bs[m][1] = *(const uint4*)(bs + 8);
    }
  };
  // the min term's A fragment: f16(dy S_j) for the 8 sub-blocks (lanes kq == 0)
  auto act_min = [&](const SkAct& r, int m) {
    h8 am = {};
    if (kq == 0) {
      const uint32_t w[8] = {r.bs[m][0].x, r.bs[m][0].y, r.bs[m][0].z, r.bs[m][0].w,
                             r.bs[m][1].x, r.bs[m][1].y, r.bs[m][1].z, r.bs[m][1].w};
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const int sv = (int)(int16_t)(w[q] & 0xFFFF) + (int)(int16_t)(w[q] >> 16);
        am[q] = (_Float16)(r.dya[m] * (float)sv);
      }
    }
    return am;
  };

  // The wave's steps run through (tile, sb) for its tiles blockIdx.x + i
  // gridDim.x and its super-blocks [sb0, sb1); the weight bytes of the next
  // two steps and the activation of the next one are in flight while a step
  // is multiplied, across tile boundaries too.
  int64_t ltile = blockIdx.x;  // the next weight load's step
  int lsb = sb0;
  auto advance = [&](int64_t& tl, int& sbx) {
    if (++sbx >= sb1) {
      sbx = sb0;
      tl += gridDim.x;
    }
  };
  SkRaw cur, nxt, nx2;
  SkAct ac, an;
  if (work && ltile < ntiles) {
    load_w(cur, ltile, lsb);
    advance(ltile, lsb);
    if (ltile < ntiles) load_w(nxt, ltile, lsb);
    advance(ltile, lsb);
    load_act(ac, sb0);
  }

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
  f4v acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int sb = sb0; sb < sb1; sb++) {
    if (ltile < ntiles) load_w(nx2, ltile, lsb);
    advance(ltile, lsb);
    const bool more = sb + 1 < sb1 || tile + gridDim.x < ntiles;
    if (more) load_act(an, sb + 1 < sb1 ? sb + 1 : sb0);
    const i4v (&a)[MT][4] = ac.a;

    // this row's scales and mins (get_scale_min_k4, utils.rs:50-60)
    const uint32_t u0 = cur.hdr.y, u1 = cur.hdr.z, u2 = cur.hdr.w;
    const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
    const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = h2f((uint16_t)(cur.hdr.x & 0xFFFF));
    const float dmin = h2f((uint16_t)(cur.hdr.x >> 16));

    i4v cacc[MT];
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int s = 2 * c + (hin ? 1 : 0);  // this lane's sub-block in chunk c
        const uint32_t sw = s < 4 ? s03 : s47;
        const uint32_t scv = (sw >> (8 * (s & 3))) & 0xFF;
        const uint32_t f = sk_dup16(pass == 0 ? scv >> 3 : scv & 7);
        const uint4& ch = sk_chunk(cur, c);
        i4v b;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t w = sk_word(ch, e);
          b[e] = (int)sk_pkmul(hin ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu, f);
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const i4v zero = {0, 0, 0, 0};
          cacc[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[m][c], b, (pass == 0 && c == 0) ? zero : cacc[m], 0, 0, 0);
        }
      }
      if (pass == 0) {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
          for (int i = 0; i < 4; i++) cacc[m][i] <<= 3;
      }
    }

    // f32 epilogue: C row i of tile m is activation row 16m + 4 kq + i
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][i] = __builtin_fmaf(ac.dy[m][i] * dw, (float)cacc[m][i], acc[m][i]);
    // min term over the 8 sub-blocks (K padded to 32: lanes 16-63 carry zeros)
    h8 bm = {};
    if (kq == 0) {
#pragma unroll
      for (int q = 0; q < 8; q++) bm[q] = (_Float16)(-dmin * (float)(((q < 4 ? m03 : m47) >> (8 * (q & 3))) & 0xFF));
    }
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(act_min(ac, m), bm, acc[m], 0, 0, 0);
    if (more) {
      cur = nxt;
      nxt = nx2;
      ac = an;
    }
  }

  // the waves' partial sums of the tile, added in wave order
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) part[wv][m][i][lane] = acc[m][i];
  __syncthreads();
  if (wv == 0) {
    const int64_t row = tile * 16 + r16;
    if (row < n_total) {
      int t;
      int64_t lrow;
      (void)tile_row(tile, t, lrow);
      float* out = tg.dst[t] + lrow;
      const int64_t ldd = tg.ldd[t];
#pragma unroll
      for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float v = part[0][m][i][lane];
#pragma unroll
          for (int w = 1; w < kSkWaves; w++) v = __fadd_rn(v, part[w][m][i][lane]);
          const int ar = 16 * m + 4 * kq + i;
          if (ar < M) out[(int64_t)ar * ldd] = v;
        }
    }
  }
  __syncthreads();  // the partials are read before the next tile's are written
  }
}

}  // namespace

int gemm_q4k_skinny_max_rows() { return 32; }

bool gemm_q4k_skinny_fits(int64_t k, int64_t rows) {
  return k % 256 == 0 && rows >= 1 && rows <= 32;
}

hipError_t launch_gemm_q4k_skinny(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, int cus,
                                  hipStream_t st) {
  // one workgroup per 16-row weight tile (measured faster than a persistent
  // grid of cus workgroups walking tiles: the tile switch drains the pipeline)
  (void)cus;
  const int64_t ntiles = (t.row_end[t.count - 1] + 15) / 16;
  const dim3 grid((unsigned)ntiles);
  const int nsb = (int)(k / 256);
  if (rows <= 16)
    gemm_q4k_skinny_kernel<1><<<grid, 64 * kSkWaves, 0, st>>>(t, nsb, p.codes, p.d, (const int16_t*)p.sums, (int)rows);
  else
    gemm_q4k_skinny_kernel<2><<<grid, 64 * kSkWaves, 0, st>>>(t, nsb, p.codes, p.d, (const int16_t*)p.sums, (int)rows);
  return hipGetLastError();
}

}  // namespace qmm
