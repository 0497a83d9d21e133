// gemm_q6k.hip — Q6_K prefill GEMM on the int8 matrix cores of gfx950, from
// 33 activation rows (fewer: gemm_q6k_skinny.hip).
//
// dst[m][n] = sum over super-blocks of  d_n dy_m sum_g sc_ng sum_{i in g} (q_ni - 32) y_mi
// is candle's Q6_K x Q8_K vec_dot (vendor/candle/candle-core/src/quantized/
// k_quants.rs:2598-2655) against the activation quantized as the reference
// quantizes it for Q6_K (BlockQ8K::from_float, :2882-2927): per-256 scale
// dy_m and int8 codes y. The reference's card path sends these products to
// its int8 MMQ kernels (quantized/cuda.rs:1005-1136).
//
// Exact integer arithmetic. A code's product with its 16-value group's int8
// scale, p = sc (q - 32), needs 14 bits; an int8 operand holds 8. Each lane
// forms 4p + 128 in a 16-bit lane (one packed multiply-add makes two), takes
// its high byte h and its low byte minus 128, l, so that 256 h + l = 4p with
// h in [-63, 64] and l in [-128, 124], and runs both bytes against the
// activation codes into two int32 tiles per output tile. Per super-block,
// 256 T_h + T_l = 4 sum p y is the reference's integer times four
// (|.| <= 256 * 127 * 16384 < 2^31), and the f32 epilogue adds
// (d_n dy_m / 4) * (256 T_h + T_l).
//
// Shape: v_mfma_i32_16x16x64_i8, activation rows on the A side, weight rows
// on the B side. A wave owns 16 weight rows and all BM = 128 activation rows
// of the workgroup tile (8 MFMA tiles). A 64-deep K-chunk c holds the groups
// 4c .. 4c+3 of the super-block: lane L takes weight row L%16 and group
// 4c + L/16, so the 16 codes a lane expands share one scale and feed 16
// MFMAs (8 tiles, two bytes each).
//
// Data movement (workgroup: kWaves waves, 128 rows x 16 kWaves weight rows):
//   - Per super-block the activation codes (128 rows x 256 B, 16-byte pieces
//     XOR-swizzled by row) and, for each weight row, the 14 aligned 16-byte
//     pieces that cover its 210-byte block (every piece holds a byte of the
//     block, so none leaves the weight's memory) reach LDS by direct
//     global-to-LDS copies, one super-block ahead into the other half of
//     double buffers. Lanes read their row's bytes back with dword reads and
//     byte alignment (blocks start at any even offset).
//   - dy of the next super-block is loaded by the first 128 threads and
//     written to LDS.
//   - Workgroups with consecutive indices share a weight tile (one per
//     activation tile), and consecutive indices are placed on one XCD, so
//     the weight bytes are read from HBM about once.
// Rows past M and weight rows past N are read as the last row (valid
// memory); their outputs are never stored.
#include <type_traits>

#include "lds_copy.h"
#include "mv_common.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128;     // activation rows of a workgroup tile
constexpr int kWin = 224;   // LDS bytes a weight row: 14 pieces of 16 bytes
constexpr int kBlock = 210;

__device__ __forceinline__ uint32_t pkmad(uint32_t a, uint32_t b, uint32_t c) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, b);
  const u16x2 z = __builtin_bit_cast(u16x2, c);
  return __builtin_bit_cast(uint32_t, (u16x2)(x * y + z));
}

// The two int8 B operands of one K-chunk from this lane's 16 codes: each
// code q = (ql nibble) | (2 bits of qh) << 4, then 4 sc q + (128 - 128 sc)
// in 16-bit lanes (even and odd bytes apart), its high bytes (bh) and its low
// bytes minus 128 (bl), in K order.
__device__ __forceinline__ void q6_operands(const uint32_t (&ql)[4], const uint32_t (&qh)[4], int nib, int qsh,
                                            uint32_t sc4, uint32_t kb, i4v& bh, i4v& bl) {
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t q = ((ql[e] >> nib) & 0x0F0F0F0Fu) | (((qh[e] >> qsh) & 0x03030303u) << 4);
    const uint32_t pe = pkmad(__builtin_amdgcn_perm(0u, q, 0x0C020C00u), sc4, kb);
    const uint32_t po = pkmad(__builtin_amdgcn_perm(0u, q, 0x0C030C01u), sc4, kb);
    bh[e] = (int)__builtin_amdgcn_perm(po, pe, 0x07030501u);
    bl[e] = (int)(__builtin_amdgcn_perm(po, pe, 0x06020400u) ^ 0x80808080u);
  }
}

// s_waitcnt that waits for all but the newest n vector-memory operations
// (global loads and global-to-LDS copies) and for nothing else.
constexpr int vmcnt_below(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

template <int kWaves, int kBuf>
__global__ __launch_bounds__(64 * kWaves, 1) void gemm_q6k_kernel(const uint8_t* __restrict__ W, int64_t N, int nsb,
                                                                   const int8_t* __restrict__ yq,
                                                                   const float* __restrict__ yd, int64_t M,
                                                                   float* __restrict__ dst, int64_t ldd, int mt,
                                                                   int remap) {
  constexpr int BN = 16 * kWaves;
  constexpr int kWInstr = BN * 14 / 64;      // 1 KB copies of the weight windows a super-block
  constexpr int kAInstr = BM * 256 / 1024;   // and of the activation tile
  constexpr int kWCopies = (kWInstr + kWaves - 1) / kWaves, kACopies = kAInstr / kWaves;
  constexpr int kCopies = kWCopies + kACopies;
  constexpr int kPerChunk = (kCopies + 3) / 4;
  static_assert(BN * 14 % 64 == 0 && kAInstr % kWaves == 0, "copy shapes");
  static_assert(kBuf == 2 || kBuf == 3, "double or triple buffers");
  // kBuf stages of the activation tile and the weight windows: the copies of
  // super-block sb + kBuf - 1 are issued while sb is computed. The loop is
  // unrolled by kBuf so every access names its stage statically (the
  // compiler then tells reads of one stage from copies into another).
  __shared__ __attribute__((aligned(16))) int8_t s_a[kBuf][BM * 256];
  // 16 spare bytes: a row's last dword read may pass its window by two
  __shared__ __attribute__((aligned(16))) uint8_t s_w[kBuf][BN * kWin + 16];
  __shared__ __attribute__((aligned(16))) float s_dy[2][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int b = (int)blockIdx.x, total = (int)gridDim.x;
  const int idx = remap ? (b & 7) * (total >> 3) + (b >> 3) : b;
  const int64_t m0 = (int64_t)(idx % mt) * BM, n0 = (int64_t)(idx / mt) * BN;
  const int64_t K = (int64_t)nsb * 256;
  const uint32_t rowbytes = (uint32_t)nsb * kBlock;

  // Weight copies: copy i moves pieces 64 i .. 64 i + 63 of the tile's
  // windows, lane L piece f = 64 i + L: window row f / 14, piece f % 14 of
  // the aligned span at or before the row's block. Byte offsets from W: the
  // host keeps N * rowbytes below 2^31.
  // Activation copies: copy i moves rows 4i .. 4i+3 of the tile; lane L
  // writes row 4i + L/16 at piece position L%16, which holds code piece
  // (L%16) ^ (row & 15). Rows past M read the last row: the host keeps
  // (M + BM) * K below 2^31.
  const uint32_t lp = lane & 15, lq = lane >> 4;
  // Every wave issues kCopies copies a super-block, without branches: a wave
  // whose last weight copy index passes kWInstr repeats its previous copy
  // (the same bytes to the same place).
  uint32_t coff[kCopies], cpiece[kWCopies];
  int cidx[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; j++) {
    if (j < kWCopies) {
      int i = wv + kWaves * j;
      i = i < kWInstr ? i : i - kWaves;
      cidx[j] = i;
      const uint32_t f = 64u * (uint32_t)i + (uint32_t)lane;
      const int64_t r = n0 + f / 14u < N ? n0 + f / 14u : N - 1;
      coff[j] = (uint32_t)r * rowbytes;  // the super-block is added per step
      cpiece[j] = 16u * (f % 14u);
    } else {
      const int i = wv + kWaves * (j - kWCopies);
      cidx[j] = i;
      const uint32_t tr = 4u * (uint32_t)i + lq;
      const int64_t r = m0 + tr < M ? m0 + tr : M - 1;
      coff[j] = (uint32_t)(r * K) + 16u * (lp ^ (tr & 15u));
    }
  }
  auto issue_one = [&](int sbi, int j, uint8_t* sw, int8_t* sa) {
    const int sb = __builtin_amdgcn_readfirstlane(sbi);
    const int i = __builtin_amdgcn_readfirstlane(cidx[j]);
    if (j < kWCopies)
      dma16(W, ((coff[j] + (uint32_t)(kBlock * sb)) & ~15u) + cpiece[j], lds_addr(sw + 1024 * i));
    else
      dma16(yq + 256 * sb, coff[j], lds_addr(sa + 1024 * i));
  };

  // dy of the tile's rows, one super-block ahead. Every thread loads and
  // stores the dy of row tid % BM (threads of one row store the same value),
  // so a step has no branch and is scheduled as one block.
  const int64_t srow = m0 + (tid & (BM - 1)) < M ? m0 + (tid & (BM - 1)) : M - 1;
  float sdy = 0.0f;
  auto load_dy = [&](int sb) { sdy = yd[srow * nsb + sb]; };
  auto store_dy = [&](int sb) { s_dy[sb & 1][tid & (BM - 1)] = sdy; };

  float acc[8][4];
#pragma unroll
  for (int m = 0; m < 8; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[m][i] = 0.0f;

  // this lane's weight row and its block's offset in its window
  const int wrow = 16 * wv + r16;
  const uint32_t wbase = (uint32_t)(n0 + wrow < N ? n0 + wrow : N - 1) * rowbytes;
  // A-operand piece of chunk c: (4c + kq) ^ r16
  const uint32_t xr = (uint32_t)r16 >> 2, xl = ((uint32_t)kq ^ (uint32_t)r16) & 3u;

#pragma unroll
  for (int s = 0; s + 1 < kBuf; s++) {
    if (s < nsb) {
#pragma unroll
      for (int j = 0; j < kCopies; j++) issue_one(s, j, s_w[s], s_a[s]);
    }
  }
  load_dy(0);
  __builtin_amdgcn_s_waitcnt(0);
  store_dy(0);
  __syncthreads();

  // Step sb: this lane's raw weight bytes and the A fragments of chunk 0,
  // then the four K-chunks, software-pipelined tile by tile: each tile's two
  // MFMAs, then its A fragment of the next chunk read into the same
  // registers, with the next chunk's B operands built under the first
  // tiles' MFMAs; in the last chunk the f32 epilogue of tile m - 1 runs
  // under tile m's MFMAs. The copies of sb + kBuf - 1 follow each chunk.
  auto step = [&](auto stage, int sb) {
    constexpr int cur = decltype(stage)::value;
    constexpr int nxt = (cur + kBuf - 1) % kBuf;
    load_dy(sb + 1 < nsb ? sb + 1 : sb);  // past the last super-block, the last one's again

    const uint8_t* win = s_w[cur] + wrow * kWin;
    const int o = (int)((wbase + (uint32_t)(kBlock * sb)) & 15u);
    uint32_t ql[2][4], qh[2][4], scw[4];
    lds_words<4>(win, o + 16 * kq, ql[0]);
    lds_words<4>(win, o + 64 + 16 * kq, ql[1]);
    lds_words<4>(win, o + 128 + 16 * (kq & 1), qh[0]);
    lds_words<4>(win, o + 160 + 16 * (kq & 1), qh[1]);
    lds_words<4>(win, o + 192, scw);
    const float dw4 = 0.25f * h2f((uint16_t)lds_u16(win, o + 208));
    const int8_t* at = s_a[cur] + r16 * 256;
    auto afrag = [&](int c, int m) -> i4v {
      return *(const i4v*)(at + 16 * 256 * m + 16 * ((((uint32_t)c ^ xr) << 2) | xl));
    };
    i4v af[8];
#pragma unroll
    for (int m = 0; m < 8; m++) af[m] = afrag(0, m);
    const float* sdyl = s_dy[sb & 1];

    // the copies of super-block sb + kBuf - 1 (past the last super-block,
    // the last one's again, into the stage no wave reads any more)
    const int sbc = sb + kBuf - 1 < nsb ? sb + kBuf - 1 : nsb - 1;
    const i4v zero = {0, 0, 0, 0};
    auto build = [&](int c, i4v& bh, i4v& bl) {
      // group 4c + kq: scale byte kq of scale word c, codes from ql half c/2
      // (low nibbles for even c) and qh bits 4 (c%2) + 2 (kq/2)
      const int sc = (int)(int8_t)(scw[c] >> (8 * kq));
      const uint32_t sc4 = ((uint32_t)(4 * sc) & 0xFFFFu) * 0x10001u;
      const uint32_t kb = ((uint32_t)(128 - 128 * sc) & 0xFFFFu) * 0x10001u;
      q6_operands(ql[c >> 1], qh[c >> 1], 4 * (c & 1), 4 * (c & 1) + 2 * (kq >> 1), sc4, kb, bh, bl);
    };
    i4v th[8], tl[8];
    // acc += (dy_m d_n / 4) (256 T_h + T_l) for tile m
    auto epi_tile = [&](int m, const float4& dy4) {
      const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = (int)(((uint32_t)th[m][i] << 8) + (uint32_t)tl[m][i]);
        acc[m][i] = __builtin_fmaf(dyv[i] * dw4, (float)t, acc[m][i]);
      }
    };
    i4v bh, bl;
    build(0, bh, bl);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      i4v nh = bh, nl = bl;
      float4 dy4[8];
#pragma unroll
      for (int m = 0; m < 8; m++) {
        th[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[m], bh, c == 0 ? zero : th[m], 0, 0, 0);
        tl[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[m], bl, c == 0 ? zero : tl[m], 0, 0, 0);
        if (c < 3) af[m] = afrag(c + 1, m);
        if (c == 3) dy4[m] = *(const float4*)&sdyl[16 * m + 4 * kq];
        if (c < 3 && m == 0) build(c + 1, nh, nl);
        if (c == 3 && m > 0) epi_tile(m - 1, dy4[m - 1]);
      }
      if (c == 3) epi_tile(7, dy4[7]);
      // the order within the chunk: each tile's MFMAs, then its next A
      // fragment (or, in the last chunk, its dy) and a share of the vector
      // work (the next chunk's B operands, or the previous tile's epilogue)
#pragma unroll
      for (int m = 0; m < 8; m++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (c < 3)
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        else
          __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = kPerChunk * c; j < kPerChunk * (c + 1) && j < kCopies; j++)
        issue_one(sbc, j, s_w[nxt], s_a[nxt]);
      bh = nh;
      bl = nl;
    }
    // the accumulators are consumed here, so the epilogue stays under the
    // last chunk's MFMAs (the compiler would otherwise sink it past the
    // barrier into the next step, as one block of vector work)
#pragma unroll
    for (int m = 0; m < 8; m++) asm volatile("" ::"v"(acc[m][0]), "v"(acc[m][1]), "v"(acc[m][2]), "v"(acc[m][3]));

    // super-block sb + 1's stage and dy have landed (with three stages, the
    // copies of sb + 2, issued after them, may still be in flight); after the
    // last super-block this stores a dy no step reads
    __builtin_amdgcn_s_waitcnt(kBuf == 3 ? vmcnt_below(kCopies) : 0);
    store_dy(sb + 1);
    // every wave is done with this stage, and the next one is complete
    __syncthreads();
  };
  for (int sb = 0; sb < nsb; sb += kBuf) {
    step(std::integral_constant<int, 0>{}, sb);
    if (sb + 1 < nsb) step(std::integral_constant<int, 1>{}, sb + 1);
    if constexpr (kBuf == 3) {
      if (sb + 2 < nsb) step(std::integral_constant<int, 2>{}, sb + 2);
    }
  }
  // the repeated copies past the last super-block land before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);

  const int64_t col = n0 + wrow;
  if (col < N) {
#pragma unroll
    for (int m = 0; m < 8; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t row = m0 + 16 * m + 4 * kq + i;
        if (row < M) dst[row * ldd + col] = acc[m][i];
      }
  }
}

}  // namespace

int gemm_q6k_min_rows() { return 33; }  // fewer rows: gemm_q6k_skinny.hip

bool gemm_q6k_fits(int64_t n, int64_t k, int64_t rows) {
  // 32-bit byte offsets inside the kernel
  return k % 256 == 0 && n * (k / 256) * kBlock + 16 < ((int64_t)1 << 31) && (rows + BM) * k < ((int64_t)1 << 31);
}

hipError_t launch_gemm_q6k(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                           int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t mt = (rows + BM - 1) / BM;
  const int nsb = (int)(k / 256);
  // 128-column tiles (8 waves) where they give every CU a workgroup, 64-column
  // tiles (4 waves) otherwise
  const bool wide = ((n + 127) / 128) * mt >= 256;
  const int64_t total = ((n + (wide ? 127 : 63)) / (wide ? 128 : 64)) * mt;
  if (total >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const int remap = total % 8 == 0;
  // the 4-wave tiles (one wave a SIMD) run three stages deep, the 8-wave ones
  // (whose second wave a SIMD hides the copies' latency) two
  if (wide)
    gemm_q6k_kernel<8, 2><<<dim3((unsigned)total), 512, 0, st>>>((const uint8_t*)w, n, nsb, p.codes, p.d, rows,
                                                                dst, ldd, (int)mt, remap);
  else
    gemm_q6k_kernel<4, 3><<<dim3((unsigned)total), 256, 0, st>>>((const uint8_t*)w, n, nsb, p.codes, p.d, rows,
                                                                dst, ldd, (int)mt, remap);
  return hipGetLastError();
}

}  // namespace qmm
