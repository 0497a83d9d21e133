// gemm_b32.hip — Q8_0, IQ4_NL and MXFP4 products of more than 8 activation
// rows on the int8 matrix cores of gfx950.
//
// dst[m][n] = sum over 32-value blocks b of (dx_nb dy_mb) sum_{i in b} x_ni y_mi
// is candle's block dot for each type (Q8_0 vendor/candle/candle-core/src/
// quantized/k_quants.rs:1294-1312, MXFP4 :517-527 with the E2M1 table doubled
// and the e8m0 scale halved, IQ4_NL :754-764) against the activation
// quantized as the reference quantizes it for them (BlockQ8_0::from_float,
// :1240-1269: per-32 f16 scale dy, int8 codes y). The reference's card path
// sends Q8_0 and MXFP4 products above its row line to its int8 MMQ kernels
// (quantized/cuda.rs:1005-1136).
//
// Each block's integer sum_i x y is exact (one v_mfma_i32_16x16x32_i8 per
// block and output tile: the 32 values of a block are exactly its K); the
// f32 epilogue adds (dx dy) * sum for every block, as the reference does.
// With one scale pair per 32 values per output, the kernel is bound by that
// vector work rather than by the matrix cores.
//
// Shape: activation rows on the A side, weight rows on the B side. A wave
// owns 16 weight rows and all BM = 128 activation rows of the workgroup tile
// (8 MFMA tiles); lane L takes weight row L%16 and values 8 (L/16) .. +7 of a
// block. K is staged 256 values (8 blocks) at a time: the activation codes
// (128 rows x 256 B, 16-byte pieces XOR-swizzled by row) and, for each weight
// row, the aligned 16-byte pieces covering its 8 blocks (clamped to the row,
// so none leaves the weight's memory) reach LDS by direct global-to-LDS
// copies, one stage ahead into the other half of double buffers; the
// activation scales of the stage are loaded by the threads. A last stage
// past the row's blocks reads repeated bytes, and its missing blocks are
// given a zero scale pair. Rows past M and weight rows past N are read as the
// last row (valid memory); their outputs are never stored.
#include <type_traits>

#include "b32_common.h"
#include "lds_copy.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));

constexpr int BM = 128;

template <int FMT>
struct B32Shape {
  static constexpr int B = Fmt32<FMT>::B;         // bytes a block
  static constexpr int SB = 8 * B;                // bytes of a row's stage
  static constexpr int P = (SB + 15 + 15) / 16;   // 16-byte pieces covering it at any offset
  static constexpr int Head = FMT == T_MXFP4 ? 1 : 2;  // scale bytes before the codes
};

// This lane's 8 int8 weights of block b (values 8 kq .. 8 kq + 7) from the
// row's staged bytes at window offset off, and the block's scale.
template <int FMT>
__device__ __forceinline__ void b32_lane(const uint8_t* win, int off, int kq, const Lut32<FMT>& lut, uint32_t q[2],
                                         float& d) {
  if constexpr (FMT == T_Q8_0) {
    d = h2f((uint16_t)lds_u16(win, off));
    lds_words<2>(win, off + 2 + 8 * kq, q);
  } else {
    if constexpr (FMT == T_MXFP4)
      d = e8m0_half(lds_u32(win, off) & 0xFF);
    else
      d = h2f((uint16_t)lds_u16(win, off));
    // values 0..15 are the low nibbles of bytes 0..15, values 16..31 the
    // high nibbles
    uint32_t n[2];
    lds_words<2>(win, off + B32Shape<FMT>::Head + 8 * (kq & 1), n);
    const int sh = 4 * (kq >> 1);
    q[0] = (uint32_t)lut16_at(n[0], sh, lut.t0, lut.t1, lut.t2, lut.t3);
    q[1] = (uint32_t)lut16_at(n[1], sh, lut.t0, lut.t1, lut.t2, lut.t3);
  }
}

template <int FMT, int kWaves>
__global__ __launch_bounds__(64 * kWaves, 1) void gemm_b32_kernel(const uint8_t* __restrict__ W, int64_t N, int nb,
                                                                   const int8_t* __restrict__ yq,
                                                                   const float* __restrict__ yd, int64_t M,
                                                                   float* __restrict__ dst, int64_t ldd, int mt,
                                                                   int remap) {
  using S = B32Shape<FMT>;
  constexpr int BN = 16 * kWaves;
  constexpr int kWin = 16 * S::P;                       // LDS bytes a weight row
  constexpr int kWInstr = (BN * S::P + 63) / 64;        // 1 KB copies of the weight windows a stage
  constexpr int kAInstr = BM * 256 / 1024;              // and of the activation tile
  constexpr int kWCopies = (kWInstr + kWaves - 1) / kWaves, kACopies = kAInstr / kWaves;
  constexpr int kCopies = kWCopies + kACopies;
  constexpr int kPerBlock = (kCopies + 7) / 8;
  constexpr int kDyPer = BM * 8 / (64 * kWaves);        // activation scales a thread loads a stage
  __shared__ __attribute__((aligned(16))) int8_t s_a[2][BM * 256];
  __shared__ __attribute__((aligned(16))) uint8_t s_w[2][kWInstr * 1024 + 16];
  // scales of the stage, block-major: s_dy[.][b][row]
  __shared__ __attribute__((aligned(16))) float s_dy[2][8][BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int b = (int)blockIdx.x, total = (int)gridDim.x;
  const int idx = remap ? (b & 7) * (total >> 3) + (b >> 3) : b;
  const int64_t m0 = (int64_t)(idx % mt) * BM, n0 = (int64_t)(idx / mt) * BN;
  const int64_t K = (int64_t)nb * 32;
  const uint32_t rowbytes = (uint32_t)nb * S::B;
  const int nst = (nb + 7) / 8;

  // Weight copies: copy i moves pieces 64 i .. 64 i + 63 of the windows, lane
  // L piece f = 64 i + L: window row f / P, piece f % P of the aligned span
  // at or before the row's stage, clamped to the piece holding the row's
  // last byte of the stage. Activation copies: copy i moves rows 4i .. 4i+3;
  // lane L writes row 4i + L/16 at piece position L%16, which holds code
  // piece (L%16) ^ (row & 15), clamped to the row's last piece. A wave whose
  // last weight copy index passes kWInstr repeats its previous copy.
  const uint32_t lp = lane & 15, lq = lane >> 4;
  uint32_t crow[kCopies], cpc[kCopies];
  int cidx[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; j++) {
    if (j < kWCopies) {
      int i = wv + kWaves * j;
      i = i < kWInstr ? i : i - kWaves;
      cidx[j] = i;
      const uint32_t f = 64u * (uint32_t)i + (uint32_t)lane;
      const uint32_t wr = f / (uint32_t)S::P < (uint32_t)BN ? f / (uint32_t)S::P : BN - 1;
      const int64_t r = n0 + wr < N ? n0 + wr : N - 1;
      crow[j] = (uint32_t)r * rowbytes;
      cpc[j] = 16u * (f % (uint32_t)S::P);
    } else {
      const int i = wv + kWaves * (j - kWCopies);
      cidx[j] = i;
      const uint32_t tr = 4u * (uint32_t)i + lq;
      const int64_t r = m0 + tr < M ? m0 + tr : M - 1;
      crow[j] = (uint32_t)(r * K);
      cpc[j] = 16u * (lp ^ (tr & 15u));
    }
  }
  auto issue_one = [&](int sti, int j, uint8_t* sw, int8_t* sa) {
    const int st = __builtin_amdgcn_readfirstlane(sti);
    const int i = __builtin_amdgcn_readfirstlane(cidx[j]);
    if (j < kWCopies) {
      const uint32_t s0 = crow[j] + (uint32_t)(S::SB * st);
      const uint32_t send = s0 + S::SB < crow[j] + rowbytes ? s0 + S::SB : crow[j] + rowbytes;
      const uint32_t a = s0 & ~15u, last = (send - 1u) & ~15u;
      const uint32_t off = a + cpc[j] < last ? a + cpc[j] : last;
      dma16(W, off, lds_addr(sw + 1024 * i));
    } else {
      const uint32_t o = (uint32_t)(256 * st) + cpc[j];
      dma16(yq, crow[j] + (o < (uint32_t)K - 16u ? o : (uint32_t)K - 16u), lds_addr(sa + 1024 * i));
    }
  };

  // activation scales: thread t loads kDyPer of the 8 x BM (block, row)
  // pairs of a stage (zero past the row's blocks)
  float sdy[kDyPer];
  auto load_dy = [&](int st) {
#pragma unroll
    for (int u = 0; u < kDyPer; u++) {
      const int e = tid + 64 * kWaves * u;
      const int row = e & (BM - 1), blk = e >> 7;
      const int64_t gr = m0 + row < M ? m0 + row : M - 1;
      const int gb = 8 * st + blk;
      const float v = yd[gr * nb + (gb < nb ? gb : nb - 1)];
      sdy[u] = gb < nb ? v : 0.0f;
    }
  };
  auto store_dy = [&](int st) {
#pragma unroll
    for (int u = 0; u < kDyPer; u++) {
      const int e = tid + 64 * kWaves * u;
      s_dy[st & 1][e >> 7][e & (BM - 1)] = sdy[u];
    }
  };

  float acc[8][4];
#pragma unroll
  for (int m = 0; m < 8; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[m][i] = 0.0f;

  const Lut32<FMT> lut;
  const int wrow = 16 * wv + r16;
  const uint32_t wbase = (uint32_t)(n0 + wrow < N ? n0 + wrow : N - 1) * rowbytes;

#pragma unroll
  for (int j = 0; j < kCopies; j++) issue_one(0, j, s_w[0], s_a[0]);
  load_dy(0);
  __builtin_amdgcn_s_waitcnt(0);
  store_dy(0);
  __syncthreads();

  // Stage st: its 8 blocks, each block's 8 MFMAs (one a tile) followed by
  // the previous block's f32 epilogue (its tiles are complete by then), with
  // the copies of stage st + 1 spread over the blocks.
  auto step = [&](auto buf, int st) {
    constexpr int cur = decltype(buf)::value, nxt = cur ^ 1;
    const int stn = st + 1 < nst ? st + 1 : st;  // past the last stage, the last one's again
    load_dy(stn);
    const uint8_t* win = s_w[cur] + wrow * kWin;
    const int o = (int)((wbase + (uint32_t)(S::SB * st)) & 15u);
    const int8_t* at = s_a[cur] + r16 * 256 + 8 * (kq & 1);
    const float(*sdyl)[BM] = s_dy[cur];
    i4v t[2][8];
    float sc[2];
    const i4v zero = {0, 0, 0, 0};
    auto epilogue = [&](int bb) {
      const i4v(&tt)[8] = t[bb & 1];
#pragma unroll
      for (int m = 0; m < 8; m++) {
        const float4 dy4 = *(const float4*)&sdyl[bb][16 * m + 4 * kq];
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[m][i] = __builtin_fmaf(sc[bb & 1] * dyv[i], (float)tt[m][i], acc[m][i]);
      }
    };
#pragma unroll
    for (int bb = 0; bb < 8; bb++) {
      uint32_t q[2];
      float dw;
      b32_lane<FMT>(win, o + S::B * bb, kq, lut, q, dw);
      // a block past the row's last gets a zero scale (its bytes are repeats)
      sc[bb & 1] = 8 * st + bb < nb ? dw : 0.0f;
      const long bq = (long)(((uint64_t)q[1] << 32) | q[0]);
      const uint32_t apiece = 16u * ((uint32_t)(2 * bb + (kq >> 1)) ^ (uint32_t)r16);
#pragma unroll
      for (int m = 0; m < 8; m++) {
        const long a = *(const long*)(at + 16 * 256 * m + apiece);
        t[bb & 1][m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq, zero, 0, 0, 0);
      }
      if (bb > 0) epilogue(bb - 1);
#pragma unroll
      for (int j = kPerBlock * bb; j < kPerBlock * (bb + 1) && j < kCopies; j++) issue_one(stn, j, s_w[nxt], s_a[nxt]);
    }
    epilogue(7);
    // stage st + 1 has landed
    __builtin_amdgcn_s_waitcnt(0);
    store_dy(st + 1);
    // every wave is done with this stage, and the next one is complete
    __syncthreads();
  };
  for (int st = 0; st < nst; st += 2) {
    step(std::integral_constant<int, 0>{}, st);
    if (st + 1 < nst) step(std::integral_constant<int, 1>{}, st + 1);
  }

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

template <int FMT>
hipError_t launch_fmt(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst, int64_t ldd,
                      hipStream_t st) {
  const int64_t mt = (rows + BM - 1) / BM;
  const int nb = (int)(k / 32);
  // 128-column tiles (8 waves) where they give every CU a workgroup, 64-column
  // tiles (4 waves) otherwise
  const bool wide = ((n + 127) / 128) * mt >= 256;
  const int64_t total = ((n + (wide ? 127 : 63)) / (wide ? 128 : 64)) * mt;
  if (total >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const int remap = total % 8 == 0;
  if (wide)
    gemm_b32_kernel<FMT, 8><<<dim3((unsigned)total), 512, 0, st>>>((const uint8_t*)w, n, nb, p.codes, p.d, rows, dst,
                                                                  ldd, (int)mt, remap);
  else
    gemm_b32_kernel<FMT, 4><<<dim3((unsigned)total), 256, 0, st>>>((const uint8_t*)w, n, nb, p.codes, p.d, rows, dst,
                                                                  ldd, (int)mt, remap);
  return hipGetLastError();
}

}  // namespace

int gemm_b32_min_rows() { return 9; }  // up to 8 rows: the decode kernels

bool gemm_b32_fits(int type, int64_t n, int64_t k, int64_t rows) {
  const int bb = type == T_Q8_0 ? 34 : type == T_IQ4_NL ? 18 : type == T_MXFP4 ? 17 : 0;
  // 32-bit byte offsets inside the kernel; a row of at least one 16-byte piece
  return bb != 0 && k % 32 == 0 && k >= 32 && n * (k / 32) * bb + 16 < ((int64_t)1 << 31) &&
         (rows + BM) * k < ((int64_t)1 << 31);
}

hipError_t launch_gemm_b32(int type, const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows,
                           float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  if (type == T_Q8_0) return launch_fmt<T_Q8_0>(w, n, k, p, rows, dst, ldd, st);
  if (type == T_IQ4_NL) return launch_fmt<T_IQ4_NL>(w, n, k, p, rows, dst, ldd, st);
  if (type == T_MXFP4) return launch_fmt<T_MXFP4>(w, n, k, p, rows, dst, ldd, st);
  return hipErrorInvalidValue;
}

}  // namespace qmm
