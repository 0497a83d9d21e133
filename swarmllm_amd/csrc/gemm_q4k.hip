// gemm_q4k.hip — Q4_K prefill GEMM on the int8 matrix cores of gfx950.
//
// dst[m][n] = sum over super-blocks sb of
//     d_n dy_m * sum_j sc_nj * sum_{i in j} q_ni y_mi  -  dmin_n dy_m * sum_j m_nj * S_mj
// the arithmetic of candle's Q4_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2031-2111) against
// the activation quantized as the reference quantizes it for Q4_K
// (BlockQ8K::from_float, :2882-2927: per-256 scale dy_m, int8 codes y, and
// S_mj = bsum_2j + bsum_2j+1 the code sums of each 32-value sub-block).
//
// Folding the 6-bit sub-block scale into the int8 operand. An int8 MFMA can
// only take sc*q (up to 945) split in two: sc = 8*sh + sl (sh, sl in 0..7),
// so sl*q and sh*q are both <= 105. Two MFMAs per K-chunk give
// C_lo = sum y*sl*q and C_hi = sum y*sh*q, and 8*C_hi + C_lo is the exact
// int32 sum_j sc_j sum_i q y of the super-block (the reference's own integer)
// with no per-sub-block work on the accumulators. The split also makes the
// dequantisation cheap: 4 nibbles packed one per byte times sl (<= 7) never
// carry out of a byte, so one packed 16-bit multiply scales 4 codes.
// Per super-block the f32 epilogue adds (d_n dy_m) * (8*C_hi + C_lo); the min
// term, a K = 8 product of f16(dy_m * S_mj) and f16(-dmin_n * m_nj), runs as one
// f16 MFMA accumulating into the same f32 tile.
//
// Tiles: a workgroup of 4 waves computes 128 x 128 outputs (2 x 2 waves of
// 64 x 64, each 2 x 2 MFMA 32x32x32 tiles), stepping K by 64 (one 64-value
// chunk of a super-block per step) through double-buffered LDS: activation
// codes, and the two weight halves sl*q and sh*q, each [row][64] padded to
// 80 bytes. Rows past M or N are zero-filled and never stored.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128, KSTEP = 64, LDK = 80;
constexpr int kThreads = 256;

struct __attribute__((aligned(16))) Smem {
  int8_t a[2][BM][LDK];
  int8_t blo[2][BN][LDK];
  int8_t bhi[2][BN][LDK];
  // per super-block, double-buffered by super-block parity
  _Float16 amin[2][BM][8];  // f16(dy_m * S_mj)
  _Float16 bmin[2][BN][8];  // f16(-dmin_n * m_nj)
  float dy[2][BM];
  float dw[2][BN];
};

// sl | sl << 16 for the packed multiply
__device__ __forceinline__ uint32_t dup16(uint32_t v) { return v | (v << 16); }

__device__ __forceinline__ uint32_t pkmul(uint32_t a, uint32_t s2) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, s2);
  return __builtin_bit_cast(uint32_t, x * y);
}

// What a thread carries from global memory for one K-step.
struct StepRegs {
  uint4 a[2];   // activation codes: pieces tid and tid + 256 of the BM x 64 tile
  uint4 q;      // Q4_K codes: 16 bytes of chunk j of weight row tid/2, half tid%2
  // once per super-block (j == 0)
  uint4 hdr;    // the weight row's super-block header
  float dy;     // activation row tid's scale (tid < BM)
  uint4 bs0, bs1;  // its 16 bsums (int16)
};

__global__ __launch_bounds__(kThreads, 1) void gemm_q4k_kernel(const uint8_t* __restrict__ W, int64_t N, int nsb,
                                                                const int8_t* __restrict__ yq,
                                                                const float* __restrict__ yd,
                                                                const int16_t* __restrict__ ybs, int64_t M,
                                                                float* __restrict__ dst, int64_t ldd) {
  __shared__ Smem sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;  // this wave's 64 x 64 block of the tile
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = (int64_t)nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;
  const int steps = nsb * 4;

  // the weight row and half this thread dequantises
  const int bn = tid >> 1, bh = tid & 1;
  const bool bvalid = n0 + bn < N;
  const uint8_t* wrow = W + (n0 + (bvalid ? bn : 0)) * rowbytes;
  // the activation pieces this thread copies: rows (tid + 256 i) / 4, 16-byte piece % 4
  auto load_step = [&](StepRegs& r, int t) {
    const int sb = t >> 2, j = t & 3;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int p = tid + kThreads * i;
      const int row = p >> 2, c = p & 3;
      r.a[i] = m0 + row < M ? *(const uint4*)(yq + (m0 + row) * K + (int64_t)sb * 256 + 64 * j + 16 * c)
                            : make_uint4(0, 0, 0, 0);
    }
    r.q = bvalid ? *(const uint4*)(wrow + (int64_t)sb * 144 + 16 + 32 * j + 16 * bh) : make_uint4(0, 0, 0, 0);
    if (j == 0) {
      r.hdr = bvalid ? *(const uint4*)(wrow + (int64_t)sb * 144) : make_uint4(0, 0, 0, 0);
      if (tid < BM) {
        const bool av = m0 + tid < M;
        r.dy = av ? yd[(m0 + tid) * nsb + sb] : 0.0f;
        const uint4* bp = (const uint4*)(ybs + (m0 + (av ? tid : 0)) * (K / 16) + (int64_t)sb * 16);
        r.bs0 = av ? bp[0] : make_uint4(0, 0, 0, 0);
        r.bs1 = av ? bp[1] : make_uint4(0, 0, 0, 0);
      }
    }
  };

  // scales of the current super-block for this thread's weight row (from the header)
  uint32_t sl2[8], sh2[8];
  auto store_step = [&](const StepRegs& r, int t) {
    const int buf = t & 1, sb = t >> 2, j = t & 3, sbuf = sb & 1;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int p = tid + kThreads * i;
      *(uint4*)&sm.a[buf][p >> 2][16 * (p & 3)] = r.a[i];
    }
    if (j == 0) {
      // 6-bit scales and mins of the 8 sub-blocks (get_scale_min_k4, utils.rs:50-60)
      const uint32_t u0 = r.hdr.y, u1 = r.hdr.z, u2 = r.hdr.w;
      const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
      const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
      const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const uint32_t sc = ((q < 4 ? s03 : s47) >> (8 * (q & 3))) & 0xFF;
        sl2[q] = dup16(sc & 7);
        sh2[q] = dup16(sc >> 3);
      }
      if (bh == 0) {
        const float d = h2f((uint16_t)(r.hdr.x & 0xFFFF)), dmin = h2f((uint16_t)(r.hdr.x >> 16));
        h8 bm;
#pragma unroll
        for (int q = 0; q < 8; q++) bm[q] = (_Float16)(-dmin * (float)(((q < 4 ? m03 : m47) >> (8 * (q & 3))) & 0xFF));
        *(h8*)&sm.bmin[sbuf][bn][0] = bm;
        sm.dw[sbuf][bn] = d;
      }
      if (tid < BM) {
        const uint32_t w[8] = {r.bs0.x, r.bs0.y, r.bs0.z, r.bs0.w, r.bs1.x, r.bs1.y, r.bs1.z, r.bs1.w};
        h8 am;
#pragma unroll
        for (int q = 0; q < 8; q++) {
          // S_q = bsum_2q + bsum_2q+1 (the two int16 of word q)
          const int s = (int)(int16_t)(w[q] & 0xFFFF) + (int)(int16_t)(w[q] >> 16);
          am[q] = (_Float16)(r.dy * (float)s);
        }
        *(h8*)&sm.amin[sbuf][tid][0] = am;
        sm.dy[sbuf][tid] = r.dy;
      }
    }
    // weight codes: 16 bytes = values l0..l0+15 of sub-blocks 2j (low nibbles)
    // and 2j+1 (high nibbles), l0 = 16*bh; k within the step: l0 + b and 32 + l0 + b
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    uint32_t lo_a[4], hi_a[4], lo_b[4], hi_b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t a = qw[i] & 0x0F0F0F0Fu, b = (qw[i] >> 4) & 0x0F0F0F0Fu;
      lo_a[i] = pkmul(a, sl2[2 * j]);
      hi_a[i] = pkmul(a, sh2[2 * j]);
      lo_b[i] = pkmul(b, sl2[2 * j + 1]);
      hi_b[i] = pkmul(b, sh2[2 * j + 1]);
    }
    const int l0 = 16 * bh;
    *(uint4*)&sm.blo[buf][bn][l0] = make_uint4(lo_a[0], lo_a[1], lo_a[2], lo_a[3]);
    *(uint4*)&sm.bhi[buf][bn][l0] = make_uint4(hi_a[0], hi_a[1], hi_a[2], hi_a[3]);
    *(uint4*)&sm.blo[buf][bn][32 + l0] = make_uint4(lo_b[0], lo_b[1], lo_b[2], lo_b[3]);
    *(uint4*)&sm.bhi[buf][bn][32 + l0] = make_uint4(hi_b[0], hi_b[1], hi_b[2], hi_b[3]);
  };

  // accumulators: per super-block int32 halves, and the f32 result
  i16v clo[2][2], chi[2][2];
  f16v acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 2; b++) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        clo[a][b][i] = 0;
        chi[a][b][i] = 0;
        acc[a][b][i] = 0.0f;
      }
    }

  StepRegs regs;
  load_step(regs, 0);
  store_step(regs, 0);
  __syncthreads();

  const int r32 = lane & 31, kh = 16 * (lane >> 5);
  for (int t = 0; t < steps; t++) {
    const int buf = t & 1;
    if (t + 1 < steps) load_step(regs, t + 1);
    // two 32-value K-chunks of the step
#pragma unroll
    for (int kc = 0; kc < 2; kc++) {
      i4v af[2], bl[2], bhv[2];
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
        af[tm] = *(const i4v*)&sm.a[buf][64 * wm + 32 * tm + r32][32 * kc + kh];
#pragma unroll
      for (int tn = 0; tn < 2; tn++) {
        bl[tn] = *(const i4v*)&sm.blo[buf][64 * wn + 32 * tn + r32][32 * kc + kh];
        bhv[tn] = *(const i4v*)&sm.bhi[buf][64 * wn + 32 * tn + r32][32 * kc + kh];
      }
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
          clo[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bl[tn], clo[tm][tn], 0, 0, 0);
          chi[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bhv[tn], chi[tm][tn], 0, 0, 0);
        }
    }
    if ((t & 3) == 3) {
      // end of a super-block: scale into the f32 result, then the min term
      const int sbuf = (t >> 2) & 1;
#pragma unroll
      for (int tn = 0; tn < 2; tn++) {
        const float dwn = sm.dw[sbuf][64 * wn + 32 * tn + r32];
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const float4 dy4 = *(const float4*)&sm.dy[sbuf][64 * wm + 32 * tm + 8 * g + 4 * (lane >> 5)];
            const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int i = 4 * g + e;
              const int tot = (chi[tm][tn][i] << 3) + clo[tm][tn][i];
              acc[tm][tn][i] = __builtin_fmaf(dyv[e] * dwn, (float)tot, acc[tm][tn][i]);
              clo[tm][tn][i] = 0;
              chi[tm][tn][i] = 0;
            }
          }
        }
      }
      h8 amf[2], bmf[2];
      const h8 z = {};
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
        amf[tm] = lane < 32 ? *(const h8*)&sm.amin[sbuf][64 * wm + 32 * tm + r32][0] : z;
#pragma unroll
      for (int tn = 0; tn < 2; tn++)
        bmf[tn] = lane < 32 ? *(const h8*)&sm.bmin[sbuf][64 * wn + 32 * tn + r32][0] : z;
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(amf[tm], bmf[tn], acc[tm][tn], 0, 0, 0);
    }
    if (t + 1 < steps) {
      // buffer (t+1)&1 was last read in step t-1, which every wave finished
      // before the barrier that ended it
      store_step(regs, t + 1);
    }
    __syncthreads();
  }

  // store
#pragma unroll
  for (int tm = 0; tm < 2; tm++)
#pragma unroll
    for (int tn = 0; tn < 2; tn++) {
      const int64_t col = n0 + 64 * wn + 32 * tn + r32;
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int64_t row = m0 + 64 * wm + 32 * tm + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row < M) dst[row * ldd + col] = acc[tm][tn][i];
      }
    }
}

}  // namespace

int gemm_q4k_min_rows() { return 9; }

hipError_t launch_gemm_q4k(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                           int64_t ldd, hipStream_t st) {
  const dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((rows + BM - 1) / BM));
  gemm_q4k_kernel<<<grid, kThreads, 0, st>>>((const uint8_t*)w, n, (int)(k / 256), p.codes, p.d,
                                             (const int16_t*)p.sums, rows, dst, ldd);
  return hipGetLastError();
}

}  // namespace qmm
