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
// so sl*q and sh*q are both <= 105. Per super-block a wave runs the eight
// 32-deep K-chunks against sh*q into its int32 tiles, shifts them left by 3,
// then runs the eight chunks again against sl*q into the same tiles: the
// result is the exact int32 sum_j sc_j sum_i q y of the super-block (the
// reference's own integer), with one set of accumulators and no
// per-sub-block work on them. 4 nibbles packed one per byte times sh or sl
// (<= 7) never carry out of a byte, so one packed 16-bit multiply scales 4
// codes. The f32 epilogue then adds (d_n dy_m) * T; the min term, a K = 8
// product of f16(dy_m * S_mj) and f16(-dmin_n * m_nj), runs as one f16 MFMA
// accumulating into the same f32 tile.
//
// Data movement, sized by what gfx950 measures (LDS reads of 16 bytes a
// lane ~236 B/clk per CU, LDS writes ~72 B/clk): nothing the weights expand
// into is written to LDS, and the raw bytes reach LDS without passing
// through registers.
//   - A workgroup of kWaves waves computes 128 rows x 32 kWaves columns,
//     each wave 128 x 32 (4 MFMA 32x32x32 tiles).
//   - Per super-block the workgroup's raw Q4_K weight bytes (144 per row)
//     and activation codes (256 per row) are copied to LDS with the direct
//     global-to-LDS loads (global_load_lds_dwordx4), one super-block ahead
//     into the other half of a double buffer. Activation rows' 16-byte
//     pieces are XOR-swizzled by row so the MFMA reads are conflict-free;
//     weight rows are stored one after another (144 bytes each), each copy
//     moving about 7 rows' contiguous bytes. (Copies of one 16-byte piece of
//     64 rows, 2304 bytes apart, touch 64 cache lines each and made the
//     kernel twice as slow on C3.)
//   - Each lane reads its weight row's header and the 16 code bytes
//     32j + 16(lane/32) of each 32-byte chunk j — exactly its MFMA B-operand
//     bytes for sub-blocks 2j (low nibbles) and 2j+1 (high nibbles) — and
//     dequantises them in registers.
//   - dy_m and f16(dy_m * S_mj) per super-block are loaded by the
//     workgroup's threads and written to LDS (2.5 KB).
// Rows past M or N are read as the last row (valid memory); their outputs
// are never stored.
#include "lds_copy.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 128;  // rows of a workgroup tile

__device__ __forceinline__ uint32_t pkmul(uint32_t a, uint32_t s2) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, s2);
  return __builtin_bit_cast(uint32_t, x * y);
}

__device__ __forceinline__ uint32_t word(const uint4& c, int e) {
  return e == 0 ? c.x : e == 1 ? c.y : e == 2 ? c.z : c.w;
}

// Raw bytes a lane reads of its weight row for one super-block.
struct WRaw {
  uint4 hdr;             // d, dmin, 12 scale bytes
  uint4 c0, c1, c2, c3;  // code bytes 32j + 16h .. +15 for j = 0..3
};

__device__ __forceinline__ const uint4& chunk(const WRaw& r, int j) {
  return j == 0 ? r.c0 : j == 1 ? r.c1 : j == 2 ? r.c2 : r.c3;
}

template <int kWaves>
__global__ __launch_bounds__(64 * kWaves, 1) void gemm_q4k_kernel(const uint8_t* __restrict__ W, int64_t N, int nsb,
                                                                   const int8_t* __restrict__ yq,
                                                                   const float* __restrict__ yd,
                                                                   const int16_t* __restrict__ ybs, int64_t M,
                                                                   float* __restrict__ dst, int64_t ldd) {
  constexpr int BN = 32 * kWaves;               // columns (weight rows) of the tile
  constexpr int kWInstr = BN * 144 / 1024;      // 1 KB copies of the weight tile per super-block
  constexpr int kAInstr = BM * 256 / 1024;      // and of the activation tile
  // Each half of each double buffer is its own object and the super-block
  // loop is unrolled by two, so every access names its buffer statically and
  // the compiler can tell reads of one half from copies into the other (it
  // would otherwise wait for the copies before every LDS read).
  __shared__ __attribute__((aligned(16))) int8_t s_a0[BM * 256], s_a1[BM * 256];
  __shared__ __attribute__((aligned(16))) uint8_t s_w0[BN * 144], s_w1[BN * 144];
  // per-super-block activation scales (written by threads, not copied)
  __shared__ __attribute__((aligned(16))) _Float16 s_amin[2][BM][8];
  __shared__ __attribute__((aligned(16))) float s_dy[2][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = (int64_t)nsb * 256;
  const uint32_t rowbytes = (uint32_t)nsb * 144;
  const int h = lane >> 5, r32 = lane & 31;

  // Weight copies: the tile is stored row by row, 144 bytes a row (9 pieces
  // of 16 bytes: piece 0 the header, pieces 1-8 the codes). Copy i = wv +
  // kWaves u moves pieces 64 i .. 64 i + 63 of the tile, lane L piece
  // f = 64 i + L, row f / 9, piece f % 9: each copy reads about 7 rows'
  // contiguous 144 bytes (a row of the tile per 9 lanes) rather than 16 bytes
  // of 64 rows. Rows past N read the last row. Byte offsets from W: the host
  // keeps N * rowbytes below 2^31.
  const uint32_t wlast = (uint32_t)(N - 1) * rowbytes;
  // Activation copies: copy i moves rows 4i .. 4i+3 of the tile; lane L
  // writes row 4i + L/16 at piece position L%16, which holds code piece
  // (L%16) ^ (row & 15) = (L%16) ^ (4 (i & 3) + L/16). Byte offsets from yq,
  // rows past M read the last row: the host keeps (M + BM) * K below 2^31.
  const uint32_t lp = lane & 15, lq = lane >> 4;
  const uint32_t arow0 = (uint32_t)((m0 + lq) * K);
  const uint32_t alast = (uint32_t)((M - 1) * K);
  const uint32_t kstep4 = (uint32_t)(4 * K);

  // A wave's copies of one super-block: kWCopies of the weight tile, then
  // kACopies of the activation tile. They are issued one per K-step of the
  // super-block before (all of a CU's copies issued at once queue in the
  // memory pipeline and hold up every wave's next instruction).
  constexpr int kWCopies = (kWInstr + kWaves - 1) / kWaves, kACopies = kAInstr / kWaves;
  constexpr int kCopies = kWCopies + kACopies;
  static_assert(kCopies <= 16, "one copy a K-step");
  // Each copy's per-lane byte offset, for super-block 0 (the super-block
  // advances the scalar base address instead).
  uint32_t coff[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; j++) {
    if (j < kWCopies) {
      const uint32_t i = (uint32_t)(wv + kWaves * j);
      const uint32_t f = 64u * i + (uint32_t)lane;
      const uint32_t r = (f * 7282u) >> 16;  // f / 9 for f < 2^14
      const uint32_t row = (uint32_t)(n0 + r) * rowbytes;
      coff[j] = (row < wlast ? row : wlast) + 16u * (f - 9u * r);
    } else {
      const int i = wv + kWaves * (j - kWCopies);
      const uint32_t row = arow0 + (uint32_t)(4 * i) * (kstep4 / 4);
      coff[j] = (row < alast ? row : alast) + 16u * (lp ^ (4u * (uint32_t)(i & 3) + lq));
    }
  }
  auto issue_one = [&](int sb, int j, uint8_t* sw, int8_t* sa) {
    if (j < kWCopies) {
      const int i = wv + kWaves * j;
      if (i < kWInstr) dma16(W + 144 * sb, coff[j], lds_addr(sw + 1024 * i));
    } else {
      const int i = wv + kWaves * (j - kWCopies);
      dma16(yq + 256 * sb, coff[j], lds_addr(sa + 1024 * i));
    }
  };
  auto issue = [&](int sb, uint8_t* sw, int8_t* sa) {
#pragma unroll
    for (int j = 0; j < kCopies; j++) issue_one(sb, j, sw, sa);
  };

  // per-super-block activation scales: thread t < 256 takes row t/2, sub-blocks 4(t%2)..+3
  const int srow = (tid & 255) >> 1, shalf = tid & 1;
  const int64_t sgr = m0 + srow < M ? m0 + srow : M - 1;
  const uint32_t doff = (uint32_t)(sgr * nsb);
  const uint32_t boff = (uint32_t)(sgr * (K / 16) + 8 * shalf);
  float sdy = 0.0f;
  uint4 sbs = make_uint4(0, 0, 0, 0);
  auto load_s = [&](int sb) {
    if (tid < 256) {
      sdy = yd[doff + (uint32_t)sb];
      sbs = *(const uint4*)(ybs + (boff + 16u * (uint32_t)sb));
    }
  };
  auto store_s = [&](int sb) {
    _Float16 (*samin)[8] = s_amin[sb & 1];
    float* sdyl = s_dy[sb & 1];
    if (tid < 256) {
      h4 am;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t w = word(sbs, q);
        const int sv = (int)(int16_t)(w & 0xFFFF) + (int)(int16_t)(w >> 16);
        am[q] = (_Float16)(sdy * (float)sv);
      }
      *(h4*)&samin[srow][4 * shalf] = am;
      if (shalf == 0) sdyl[srow] = sdy;
    }
  };

  f16v acc[4];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[t][i] = 0.0f;

  issue(0, s_w0, s_a0);
  load_s(0);
  __builtin_amdgcn_s_waitcnt(0);
  store_s(0);
  __syncthreads();

  // The f32 epilogue of super-block sb: acc += (dy_m d_n) * T, then the min
  // term f16(dy_m S_mj) x f16(-dmin_n m_nj) over the 8 sub-blocks (K padded
  // to 16: lanes 32-63 carry zeros).
  auto epilogue = [&](const i16v* c, int sb, float dw, float dmin, uint32_t m03, uint32_t m47) {
    const float* sdyl = s_dy[sb & 1];
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 dy4 = *(const float4*)&sdyl[32 * t + 8 * g + 4 * h];
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * g + e;
          acc[t][i] = __builtin_fmaf(dyv[e] * dw, (float)c[t][i], acc[t][i]);
        }
      }
    }
    h8 bm = {};
    if (h == 0) {
#pragma unroll
      for (int q = 0; q < 8; q++) bm[q] = (_Float16)(-dmin * (float)(((q < 4 ? m03 : m47) >> (8 * (q & 3))) & 0xFF));
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
      h8 am = {};
      if (h == 0) am = *(const h8*)&s_amin[sb & 1][32 * t + r32][0];
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, acc[t], 0, 0, 0);
    }
  };
  i16v c[4];

  const int wrow_lds = (32 * wv + r32) * 144;  // this lane's weight row in the tile
  // one super-block from buffer half (sw, sa, samin, sdyl), the next one's
  // copies into the other half
  auto step = [&](int sb, const uint8_t* sw, const int8_t* sa, uint8_t* nw, int8_t* na) {
    const bool more = sb + 1 < nsb;
    if (more) load_s(sb + 1);

    WRaw cur;
    {
      // rows 144 bytes (36 dwords) apart: the 16-byte reads of 16 lanes
      // cover the 64 banks once
      const uint8_t* wl = sw + wrow_lds;
      cur.hdr = *(const uint4*)wl;
      cur.c0 = *(const uint4*)(wl + 16 * (1 + h));
      cur.c1 = *(const uint4*)(wl + 16 * (3 + h));
      cur.c2 = *(const uint4*)(wl + 16 * (5 + h));
      cur.c3 = *(const uint4*)(wl + 16 * (7 + h));
    }
    // this row's scales and mins (get_scale_min_k4, utils.rs:50-60)
    const uint32_t u0 = cur.hdr.y, u1 = cur.hdr.z, u2 = cur.hdr.w;
    const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
    const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = h2f((uint16_t)(cur.hdr.x & 0xFFFF));
    const float dmin = h2f((uint16_t)(cur.hdr.x >> 16));

    // the int32 super-block sums: 8 * sum(y * sh q) + sum(y * sl q).
    // A-operand piece of K-chunk kc: (2kc + h) ^ (r32 & 15) = 2 (kc ^ xh) + hl
    const int xh = (r32 & 15) >> 1;
    const int8_t* at = sa + r32 * 256 + 16 * (h ^ (r32 & 1));
    // The B operand of K-chunk kc of pass p: this lane's 16 code bytes of
    // chunk kc/2 (low nibbles for even kc, high for odd) times sh or sl,
    // the factor byte placed in both 16-bit halves by one byte permute.
    const uint32_t sh03 = (s03 >> 3) & 0x07070707u, sl03 = s03 & 0x07070707u;
    const uint32_t sh47 = (s47 >> 3) & 0x07070707u, sl47 = s47 & 0x07070707u;
    auto make_b = [&](int pass, int kc) {
      const uint32_t sw = pass == 0 ? (kc < 4 ? sh03 : sh47) : (kc < 4 ? sl03 : sl47);
      const uint32_t k = (uint32_t)(kc & 3);
      const uint32_t f = __builtin_amdgcn_perm(0u, sw, 0x0C000C00u | (k << 16) | k);
      const uint4& ch = chunk(cur, kc >> 1);
      i4v b;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t w = word(ch, e);
        b[e] = (int)pkmul((kc & 1) ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu, f);
      }
      return b;
    };
    auto load_a = [&](int kc, i4v (&a)[4]) {
#pragma unroll
      for (int t = 0; t < 4; t++) a[t] = *(const i4v*)(at + 32 * t * 256 + 32 * (kc ^ xh));
    };
    // Software-pipelined by one K-chunk, tile by tile: tile t's A fragment
    // of the next chunk is read right after tile t's MFMA has taken the
    // current one (three MFMAs before it is needed), the next chunk's B
    // operand is built under the MFMAs, and at the start of the second pass
    // each tile is shifted just before its first MFMA of that pass.
    const int8_t* const at_t[4] = {at, at + 32 * 256, at + 64 * 256, at + 96 * 256};
    // The matrix loop runs at a higher issue priority than the epilogue:
    // while one wave of a SIMD is in its f32 epilogue, the other's MFMAs and
    // operand work go first and keep the matrix unit fed.
    __builtin_amdgcn_s_setprio(1);
    i4v bq = make_b(0, 0);
    i4v af[4];
    load_a(0, af);
#pragma unroll
    for (int step = 0; step < 16; step++) {
      const int ns = step + 1;
      i4v bn = bq;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        if (step == 8) {
#pragma unroll
          for (int i = 0; i < 16; i++) c[t][i] <<= 3;
        }
        const i16v zero = {};
        c[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[t], bq, step == 0 ? zero : c[t], 0, 0, 0);
        if (ns < 16) af[t] = *(const i4v*)(at_t[t] + 32 * ((ns & 7) ^ xh));
        if (t == 1 && ns < 16) bn = make_b(ns >> 3, ns & 7);
      }
      // The copies of super-block sb + 1 (at the last super-block, the last
      // one's again, into the half no wave reads any more: no branch in the
      // chunk's block).
      if (step < kCopies) issue_one(more ? sb + 1 : sb, step, nw, na);
      bq = bn;
      // The order within the chunk: each MFMA, then its tile's next
      // fragment read; the next B operand after the second MFMA; the
      // second pass's shifts each before their tile's MFMA.
#pragma unroll
      for (int t = 0; t < 4; t++) {
        if (step == 8) __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (ns < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (t == 1 && ns < 16) __builtin_amdgcn_sched_group_barrier(0x002, 13, 0);
      }
      // keep each K-chunk's work in its block (hoisting the operand loads of
      // every chunk would hold 64 fragments in registers)
      __builtin_amdgcn_sched_barrier(0);
    }

    __builtin_amdgcn_s_setprio(0);
    epilogue(c, sb, dw, dmin, m03, m47);

    if (more) {
      // the next super-block's tiles and scales have landed
      __builtin_amdgcn_s_waitcnt(0);
      store_s(sb + 1);
    }
    // every wave is done with this buffer, and the next one is complete
    __syncthreads();
  };
  for (int sb = 0; sb < nsb; sb += 2) {
    step(sb, s_w0, s_a0, s_w1, s_a1);
    if (sb + 1 < nsb) step(sb + 1, s_w1, s_a1, s_w0, s_a0);
  }
  // the last super-block's repeated copies land before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);

  const int64_t col = n0 + 32 * wv + r32;
  if (col < N) {
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int64_t row = m0 + 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
        if (row < M) dst[row * ldd + col] = acc[t][i];
      }
  }
}

constexpr int kWavesWide = 8, kWavesNarrow = 4;

}  // namespace

int gemm_q4k_min_rows() { return 33; }  // fewer rows: gemm_q4k_skinny.hip

bool gemm_q4k_fits(int64_t n, int64_t k, int64_t rows) {
  // 32-bit byte offsets inside the kernel
  return k % 256 == 0 && n * (k / 256) * 144 < ((int64_t)1 << 31) && (rows + BM) * k < ((int64_t)1 << 31);
}

hipError_t launch_gemm_q4k(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                           int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  // 256-column tiles where they give the grid at least one workgroup per
  // CU-sized share, 128-column tiles otherwise
  const int64_t mt = (rows + BM - 1) / BM;
  const bool wide = ((n + 255) / 256) * mt >= 192;
  const int nsb = (int)(k / 256);
  if (wide) {
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)mt);
    gemm_q4k_kernel<kWavesWide><<<grid, 64 * kWavesWide, 0, st>>>((const uint8_t*)w, n, nsb, p.codes, p.d,
                                                                  (const int16_t*)p.sums, rows, dst, ldd);
  } else {
    const dim3 grid((unsigned)((n + 127) / 128), (unsigned)mt);
    gemm_q4k_kernel<kWavesNarrow><<<grid, 64 * kWavesNarrow, 0, st>>>((const uint8_t*)w, n, nsb, p.codes, p.d,
                                                                      (const int16_t*)p.sums, rows, dst, ldd);
  }
  return hipGetLastError();
}

}  // namespace qmm
