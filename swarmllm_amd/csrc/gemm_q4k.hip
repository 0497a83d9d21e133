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
// Tiles: a workgroup of 8 waves computes 128 x 128 outputs (2 x 4 waves of
// 64 x 32, each 2 x 1 MFMA 32x32x32 tiles; two waves per SIMD, so one's
// scaling work runs beside the other's matrix work), stepping K by one
// super-block:
// its activation codes and the two weight halves sl*q and sh*q go to LDS
// ([row][256] padded to 272 bytes), and the next super-block's bytes load
// into registers while this one is multiplied (~3000 cycles of work between
// a load and its use). Rows past M or N are zero-filled and never stored.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128, LDK = 256 + 16;  // one super-block of K per step, rows padded
constexpr int kWavesM = 2, kWavesN = 4;             // waves of 64 x 32 outputs
constexpr int kThreads = 64 * kWavesM * kWavesN;    // 512

struct __attribute__((aligned(16))) Smem {
  int8_t a[BM][LDK];
  int8_t blo[BN][LDK];
  int8_t bhi[BN][LDK];
  _Float16 amin[BM][8];  // f16(dy_m * S_mj)
  _Float16 bmin[BN][8];  // f16(-dmin_n * m_nj)
  float dy[BM];
  float dw[BN];
};

// sl | sl << 16 for the packed multiply
__device__ __forceinline__ uint32_t dup16(uint32_t v) { return v | (v << 16); }

__device__ __forceinline__ uint32_t pkmul(uint32_t a, uint32_t s2) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, s2);
  return __builtin_bit_cast(uint32_t, x * y);
}

// What a thread carries from global memory for one super-block. Rows past M
// or N are read as the last row (valid memory); their outputs are never stored.
struct StepRegs {
  uint4 a[4];   // activation codes: pieces tid + 512 i of the BM x 256 tile (16 per row)
  uint4 hdr;    // header of weight row tid/4
  uint4 q[2];   // its code bytes 32*(tid%4) .. +31 (chunk tid%4)
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
  const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / kWavesN, wn = wv % kWavesN;  // this wave's 64 x 32 block of the tile
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = (int64_t)nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;

  // the weight row and chunk this thread dequantises
  const int bn = tid >> 2, bj = tid & 3;
  const int64_t wr = n0 + bn < N ? n0 + bn : N - 1;
  const uint8_t* wrow = W + wr * rowbytes;
  const int64_t ar = m0 + tid < M ? m0 + tid : M - 1;  // activation row of the scale loads (tid < BM)
  const int8_t* arow[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int p = tid + kThreads * i;
    const int64_t r = m0 + (p >> 4) < M ? m0 + (p >> 4) : M - 1;
    arow[i] = yq + r * K + 16 * (p & 15);
  }

  auto load_sb = [&](StepRegs& r, int sb) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.a[i] = *(const uint4*)(arow[i] + (int64_t)sb * 256);
    const uint8_t* blk = wrow + (int64_t)sb * 144;
    r.hdr = *(const uint4*)blk;
    r.q[0] = *(const uint4*)(blk + 16 + 32 * bj);
    r.q[1] = *(const uint4*)(blk + 32 + 32 * bj);
    if (tid < BM) {
      r.dy = yd[ar * nsb + sb];
      const uint4* bp = (const uint4*)(ybs + ar * (K / 16) + (int64_t)sb * 16);
      r.bs0 = bp[0];
      r.bs1 = bp[1];
    }
  };

  auto store_sb = [&](const StepRegs& r) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int p = tid + kThreads * i;
      *(uint4*)&sm.a[p >> 4][16 * (p & 15)] = r.a[i];
    }
    // 6-bit scales and mins of the 8 sub-blocks (get_scale_min_k4, utils.rs:50-60)
    const uint32_t u0 = r.hdr.y, u1 = r.hdr.z, u2 = r.hdr.w;
    const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
    const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    if (bj == 0) {
      const float d = h2f((uint16_t)(r.hdr.x & 0xFFFF)), dmin = h2f((uint16_t)(r.hdr.x >> 16));
      h8 bm;
#pragma unroll
      for (int q = 0; q < 8; q++) bm[q] = (_Float16)(-dmin * (float)(((q < 4 ? m03 : m47) >> (8 * (q & 3))) & 0xFF));
      *(h8*)&sm.bmin[bn][0] = bm;
      sm.dw[bn] = d;
    }
    if (tid < BM) {
      const uint32_t w[8] = {r.bs0.x, r.bs0.y, r.bs0.z, r.bs0.w, r.bs1.x, r.bs1.y, r.bs1.z, r.bs1.w};
      h8 am;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        // S_q = bsum_2q + bsum_2q+1 (the two int16 of word q)
        const int sv = (int)(int16_t)(w[q] & 0xFFFF) + (int)(int16_t)(w[q] >> 16);
        am[q] = (_Float16)(r.dy * (float)sv);
      }
      *(h8*)&sm.amin[tid][0] = am;
      sm.dy[tid] = r.dy;
    }
    // chunk j = bj: code bytes 32j + 16i (i = 0, 1 -> offset l0 = 16i); low
    // nibbles are values 64j + l0 + b (sub-block 2j), high 64j + 32 + l0 + b
    const int j = bj;
    const uint32_t sw = j < 2 ? s03 : s47;
    const uint32_t sca = (sw >> (16 * (j & 1))) & 0xFF, scb = (sw >> (16 * (j & 1) + 8)) & 0xFF;
    const uint32_t sla = dup16(sca & 7), sha = dup16(sca >> 3), slb = dup16(scb & 7), shb = dup16(scb >> 3);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int l0 = 16 * i;
      const uint32_t qw[4] = {r.q[i].x, r.q[i].y, r.q[i].z, r.q[i].w};
      uint32_t lo_a[4], hi_a[4], lo_b[4], hi_b[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t a = qw[e] & 0x0F0F0F0Fu, b = (qw[e] >> 4) & 0x0F0F0F0Fu;
        lo_a[e] = pkmul(a, sla);
        hi_a[e] = pkmul(a, sha);
        lo_b[e] = pkmul(b, slb);
        hi_b[e] = pkmul(b, shb);
      }
      *(uint4*)&sm.blo[bn][64 * j + l0] = make_uint4(lo_a[0], lo_a[1], lo_a[2], lo_a[3]);
      *(uint4*)&sm.bhi[bn][64 * j + l0] = make_uint4(hi_a[0], hi_a[1], hi_a[2], hi_a[3]);
      *(uint4*)&sm.blo[bn][64 * j + 32 + l0] = make_uint4(lo_b[0], lo_b[1], lo_b[2], lo_b[3]);
      *(uint4*)&sm.bhi[bn][64 * j + 32 + l0] = make_uint4(hi_b[0], hi_b[1], hi_b[2], hi_b[3]);
    }
  };

  f16v acc[2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[a][i] = 0.0f;

  StepRegs regs;
  load_sb(regs, 0);
  const int r32 = lane & 31, kh = 16 * (lane >> 5);
  const int nrow = 32 * wn + r32;  // this lane's weight row (output column) in the tile
  for (int sb = 0; sb < nsb; sb++) {
    // every wave is done with the previous super-block's LDS
    if (sb > 0) __syncthreads();
    store_sb(regs);
    __syncthreads();
    // the next super-block's bytes travel while this one is multiplied
    if (sb + 1 < nsb) load_sb(regs, sb + 1);

    i16v clo[2], chi[2];
#pragma unroll
    for (int kc = 0; kc < 8; kc++) {
      const i4v bl = *(const i4v*)&sm.blo[nrow][32 * kc + kh];
      const i4v bhv = *(const i4v*)&sm.bhi[nrow][32 * kc + kh];
#pragma unroll
      for (int tm = 0; tm < 2; tm++) {
        const i4v af = *(const i4v*)&sm.a[64 * wm + 32 * tm + r32][32 * kc + kh];
        const i16v zero = {};
        clo[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bl, kc ? clo[tm] : zero, 0, 0, 0);
        chi[tm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bhv, kc ? chi[tm] : zero, 0, 0, 0);
      }
    }
    // scale the super-block's integers into the f32 result, then the min term
    const float dwn = sm.dw[nrow];
#pragma unroll
    for (int tm = 0; tm < 2; tm++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 dy4 = *(const float4*)&sm.dy[64 * wm + 32 * tm + 8 * g + 4 * (lane >> 5)];
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * g + e;
          const int tot = (chi[tm][i] << 3) + clo[tm][i];
          acc[tm][i] = __builtin_fmaf(dyv[e] * dwn, (float)tot, acc[tm][i]);
        }
      }
    }
    const h8 z = {};
    const h8 bmf = lane < 32 ? *(const h8*)&sm.bmin[nrow][0] : z;
#pragma unroll
    for (int tm = 0; tm < 2; tm++) {
      const h8 amf = lane < 32 ? *(const h8*)&sm.amin[64 * wm + 32 * tm + r32][0] : z;
      acc[tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(amf, bmf, acc[tm], 0, 0, 0);
    }
  }

  // store
  const int64_t col = n0 + nrow;
  if (col < N) {
#pragma unroll
    for (int tm = 0; tm < 2; tm++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int64_t row = m0 + 64 * wm + 32 * tm + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row < M) dst[row * ldd + col] = acc[tm][i];
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
