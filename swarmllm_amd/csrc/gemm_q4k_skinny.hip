// gemm_q4k_skinny.hip — Q4_K products of a few activation rows (speculative
// verification widths: 4 to 32) on the int8 matrix cores of gfx950.
//
// The arithmetic is candle's Q4_K x Q8_K vec_dot
// (vendor/candle/candle-core/src/quantized/k_quants.rs:2031-2111) with the
// inner sums as matrix-core products: per super-block the exact int32
//   T    = sum_j sc_j sum_{32} q y     (two int8 MFMA passes over the codes
//                                       with the 6-bit scale split
//                                       sc = 8 sh + sl: sh q and sl q fit int8)
//   Tmin = sum_j m_j sum_{32} y        (one int8 MFMA pass with m_j broadcast
//                                       over its sub-block: the reference's
//                                       sum of bsums times mins, exactly)
// then accD += (d dy) T and accM += (dmin dy) Tmin in f32; a row's result
// is accD - accM. It takes the products the reference sends to its int8 MMQ
// from 4 rows on weights of 2 MiB or more (mmq_takes_few_rows,
// quantized/cuda.rs:790-839).
//
// Shape: v_mfma_i32_16x16x64_i8 with the activation rows on the A side (M
// padded to 16 or 32 rows: MT tiles of 16) and 16 weight rows on the B side.
// A workgroup owns NB tiles of 16 weight rows; its kWaves waves split the
// super-blocks of K and add their partial sums of the tiles through LDS in
// wave order (deterministic). A wave streams its super-blocks of the
// workgroup's rows: per super-block the 16 NB x 144 bytes as contiguous
// 16-byte pieces (each byte loaded once), the next two super-blocks' pieces
// in flight in registers, each written to the wave's LDS buffer and read
// back in the MFMA operand layout. Lane L of a wave holds weight row L%16 of
// a tile and, of 64-deep K-chunk c, the 16 code bytes 32c + 16((L/16)%2):
// low nibbles for L/16 < 2, high nibbles otherwise. Its activation fragments
// (row L%16 of a 16-row tile, values 64c + 16(L/16) .. +15) come straight
// from the quantized planes (cache-resident), one super-block ahead, and are
// used for all NB weight tiles.
//
// One launch covers up to kMaxTargets weights sharing the activation (q/k/v,
// gate/up): their rows are numbered one after another. Rows past a target's
// end, and activation rows past M, are read clamped and never stored.
#include "lds_copy.h"
#include "mv_common.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t sk_dup16(uint32_t v) { return v | (v << 16); }

__device__ __forceinline__ uint32_t sk_pkmul(uint32_t a, uint32_t s2) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, s2);
  return __builtin_bit_cast(uint32_t, x * y);
}

__device__ __forceinline__ uint32_t sk_word(const uint4& c, int e) {
  return e == 0 ? c.x : e == 1 ? c.y : e == 2 ? c.z : c.w;
}

// The pieces of one super-block of a workgroup's 16 NB rows that a lane
// loads: piece p = lane + 64 t is 16-byte piece p % 9 of row p / 9.
template <int NB>
struct SkPieces {
  static constexpr int P = 16 * NB * 9;
  static constexpr int L = (P + 63) / 64;
  uint4 v[L];
};

template <int MT>
struct SkAct {
  i4v a[MT][4];     // A fragments, K-chunks 0..3
  float dy[MT][4];  // activation scales of the C rows 16 mt + 4 (L/16) + i
};

template <int MT, int NB, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void gemm_q4k_skinny_kernel(MvTargets tg, int nsb,
                                                                      const int8_t* __restrict__ yq,
                                                                      const float* __restrict__ yd, int M) {
  constexpr int ROWS = 16 * NB;
  using Pieces = SkPieces<NB>;
  constexpr int L = Pieces::L;
  // the wave's buffer: one super-block of the rows; after the loop, its
  // partial sums [NB][MT][4][64] for the reduction
  constexpr int kBuf = ROWS * 144 > NB * MT * 4 * 64 * 4 ? ROWS * 144 : NB * MT * 4 * 64 * 4;
  __shared__ __attribute__((aligned(16))) uint8_t sbuf[kWaves][kBuf];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const bool hin = kq >= 2;      // this lane's K-slices are high nibbles
  const int hb = 16 * (kq & 1);  // byte offset of its 16 code bytes within a 32-byte chunk
  const int64_t K = (int64_t)nsb * 256;
  const int64_t rowbytes = (int64_t)nsb * 144;
  const int64_t n_total = tg.row_end[tg.count - 1];
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  uint8_t* const buf = sbuf[wv];

  // the wave's super-blocks
  const int per = (nsb + kWaves - 1) / kWaves;
  const int sb0 = wv * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;

  auto row_at = [&](int64_t R, int& t, int64_t& lrow) {
    R = R < n_total ? R : n_total - 1;
    t = 0;
#pragma unroll
    for (int i = 0; i < kMaxTargets - 1; i++)
      if (i < tg.count - 1 && R >= tg.row_end[i]) t = i + 1;
    lrow = R - (t ? tg.row_end[t - 1] : 0);
  };

  // the lane's pieces: their source in super-block 0 (the rows stay fixed)
  const uint8_t* src[L];
#pragma unroll
  for (int t = 0; t < L; t++) {
    const int p = lane + 64 * t;
    const int pp = p < Pieces::P ? p : Pieces::P - 1;
    int tt;
    int64_t lr;
    row_at(row0 + pp / 9, tt, lr);
    src[t] = (const uint8_t*)tg.w[tt] + lr * rowbytes + 16 * (pp % 9);
  }
  auto load_w = [&](Pieces& pc, int sb) {
#pragma unroll
    for (int t = 0; t < L; t++) pc.v[t] = ld_stream16(src[t] + (int64_t)sb * 144);
  };
  // every lane writes (lanes past the pieces rewrite the last piece, which
  // they loaded too): no branch, so the loads' wait counts stay exact
  auto stage_w = [&](const Pieces& pc) {
#pragma unroll
    for (int t = 0; t < L; t++) {
      const int p = lane + 64 * t;
      *(uint4*)(buf + 16 * (p < Pieces::P ? p : Pieces::P - 1)) = pc.v[t];
    }
  };

  // activation rows of this lane's A fragments and of its C rows (clamped to M - 1)
  int64_t arow[MT];
  int64_t crow[MT][4];
#pragma unroll
  for (int m = 0; m < MT; m++) {
    arow[m] = 16 * m + r16 < M ? 16 * m + r16 : M - 1;
#pragma unroll
    for (int i = 0; i < 4; i++) crow[m][i] = 16 * m + 4 * kq + i < M ? 16 * m + 4 * kq + i : M - 1;
  }
  auto load_a = [&](SkAct<MT>& r, int sb) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
      for (int c = 0; c < 4; c++) r.a[m][c] = *(const i4v*)(yq + arow[m] * K + (int64_t)sb * 256 + 64 * c + 16 * kq);
#pragma unroll
      for (int i = 0; i < 4; i++) r.dy[m][i] = yd[crow[m][i] * nsb + sb];
    }
  };

  float accD[NB][MT][4], accM[NB][MT][4];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) accD[b][m][i] = accM[b][m][i] = 0.0f;

  // one super-block from the buffer: both passes, the min pass, the f32 epilogue
  auto compute = [&](const SkAct<MT>& act) {
    // each f32 operation rounded on its own (no contraction into fma)
#pragma clang fp contract(off)
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const uint8_t* rowp = buf + (16 * b + r16) * 144;
      const uint4 hdr = *(const uint4*)rowp;
      uint4 code[4];
#pragma unroll
      for (int c = 0; c < 4; c++) code[c] = *(const uint4*)(rowp + 16 + 32 * c + hb);
      // scales and mins (get_scale_min_k4, utils.rs:50-60)
      const uint32_t u0 = hdr.y, u1 = hdr.z, u2 = hdr.w;
      const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
      const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
      const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
      const float dw = h2f((uint16_t)(hdr.x & 0xFFFF));
      const float dmin = h2f((uint16_t)(hdr.x >> 16));

      i4v T[MT], Tm[MT];
      const i4v zero = {0, 0, 0, 0};
#pragma unroll
      for (int pass = 0; pass < 2; pass++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int s = 2 * c + (hin ? 1 : 0);  // this lane's sub-block in chunk c
          const uint32_t scv = ((s < 4 ? s03 : s47) >> (8 * (s & 3))) & 0xFF;
          const uint32_t f = sk_dup16(pass == 0 ? scv >> 3 : scv & 7);
          i4v bq;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t w = sk_word(code[c], e);
            bq[e] = (int)sk_pkmul(hin ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu, f);
          }
#pragma unroll
          for (int m = 0; m < MT; m++)
            T[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(act.a[m][c], bq, (pass == 0 && c == 0) ? zero : T[m], 0, 0, 0);
        }
        if (pass == 0) {
#pragma unroll
          for (int m = 0; m < MT; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) T[m][i] <<= 3;
        }
      }
      // the mins: m_j over its 32 values, against the same fragments
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int s = 2 * c + (hin ? 1 : 0);
        const uint32_t mv = ((s < 4 ? m03 : m47) >> (8 * (s & 3))) & 0xFF;
        const int mb = (int)(mv * 0x01010101u);
        const i4v bm = {mb, mb, mb, mb};
#pragma unroll
        for (int m = 0; m < MT; m++)
          Tm[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(act.a[m][c], bm, c == 0 ? zero : Tm[m], 0, 0, 0);
      }
      // f32: C row i of tile m is activation row 16m + 4 (L/16) + i
#pragma unroll
      for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          accD[b][m][i] = accD[b][m][i] + (dw * act.dy[m][i]) * (float)T[m][i];
          accM[b][m][i] = accM[b][m][i] + (dmin * act.dy[m][i]) * (float)Tm[m][i];
        }
    }
  };

  // The loop, unrolled by two so the register buffers keep their registers.
  // A step stages super-block sb, issues the weight loads of sb + 2,
  // computes sb and then reloads the activation registers it just used with
  // sb + 2. A wave's loads complete in issue order, so a wait for an
  // activation load also waits for every weight load issued before it:
  // loading the activation of sb + 1 before computing sb (as one might)
  // would make compute(sb + 1) wait for the weights of sb + 2 as well, and
  // only one step of weights would stay in flight. Issued this way, both the
  // next step's and the one after's weights are in flight while a
  // super-block is computed (C5's few-row products take the same time either
  // way: their bound is not the depth of the loads). The main loop runs while
  // both of its steps have all their loads, which it then issues
  // unconditionally (a load issued on one path and not another makes the
  // compiler wait for every load in flight); the last steps follow it,
  // loading only what remains.
  Pieces pa, pb;
  SkAct<MT> aa, ab;
  if (sb0 < sb1) {
    load_w(pa, sb0);
    load_a(aa, sb0);
    if (sb0 + 1 < sb1) {
      load_w(pb, sb0 + 1);
      load_a(ab, sb0 + 1);
    }
  }
  // The matrix work runs at a raised wave priority: while the other wave of
  // a SIMD stages and issues loads, this one's MFMAs and operand work go
  // first (C5 at 8 rows: 7.27-7.31 -> 7.18 ms a forward).
  auto step_full = [&](Pieces& pc, SkAct<MT>& cur, int sb) {
    wave_lds_sync();  // the previous super-block's reads are done
    stage_w(pc);
    load_w(pc, sb + 2);
    wave_lds_sync();
    __builtin_amdgcn_s_setprio(1);
    compute(cur);
    __builtin_amdgcn_s_setprio(0);
    load_a(cur, sb + 2);
  };
  auto step_tail = [&](Pieces& pc, SkAct<MT>& cur, int sb) {
    wave_lds_sync();
    stage_w(pc);
    if (sb + 2 < sb1) load_w(pc, sb + 2);
    wave_lds_sync();
    compute(cur);
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

  // the waves' partial sums of the tiles, added in wave order
  wave_lds_sync();
  float* part = (float*)buf;
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) part[((b * MT + m) * 4 + i) * 64 + lane] = __fsub_rn(accD[b][m][i], accM[b][m][i]);
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int64_t R = row0 + 16 * b + r16;
      if (R >= n_total) continue;
      int t;
      int64_t lrow;
      row_at(R, t, lrow);
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

template <int MT, int NB, int W>
hipError_t launch_sk(const MvTargets& t, int nsb, const ActPlanes& p, int64_t rows, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t n_total = t.row_end[t.count - 1];
  const dim3 grid((unsigned)((n_total + 16 * NB - 1) / (16 * NB)));
  gemm_q4k_skinny_kernel<MT, NB, W><<<grid, 64 * W, 0, st>>>(t, nsb, p.codes, p.d, (int)rows);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// The same product for wide weights, its weights and activation copied
// straight to LDS (global_load_lds), SBS super-blocks of each row a stage,
// two stages in flight. A wave owns a 16-row tile over the whole of K (no sum
// across waves); the 4 waves of a workgroup share each stage's activation.
// The copies read SBS x 144 contiguous bytes of a row at once, which HBM
// streams faster than the 144-byte pieces of the register-staged kernel
// (plain reads of C5's gate+up: 4.3 TB/s in 144-byte pieces of 32 rows,
// 5.8 in 288-byte pieces of 16). Tiles are numbered weight after weight, so
// a tile never spans two weights; a ragged last tile reads its weight's last
// row again and stores only its own rows.
// ---------------------------------------------------------------------------
template <int MT, int SBS>
struct SkDma {
  static constexpr int kWSlots = 9 * SBS + 1;                  // 16-byte slots a staged weight row (+1: banks)
  static constexpr int kWCopies = (16 * kWSlots + 63) / 64;    // a wave's weight copies a stage
  static constexpr int kWStage = kWCopies * 1024;
  static constexpr int AR = 16 * MT;                           // activation rows staged
  static constexpr int kASlots = 16 * SBS + 1;                 // slots a staged activation row (+1: banks)
  static constexpr int kACopies = (AR * kASlots + 255) / 256;  // a wave's activation copies a stage
  static constexpr int kAStage = 4 * kACopies * 1024;
  static constexpr int kDStage = 4 * 256;                      // dy: one dword copy a wave (AR x SBS used)
  static constexpr int kStage = 4 * kWStage + kAStage + kDStage;
  static constexpr int kCopies = kWCopies + kACopies + 1;      // copies a wave issues a stage
  static_assert(AR * SBS <= 256, "dy of a stage fits the four dword copies");
  static_assert(kCopies <= 63, "vmcnt");
};

struct SkDmaArgs {
  MvTargets tg;
  int tile_end[kMaxTargets];  // 16-row tiles of weights 0..t
};

// A workgroup barrier that waits for nothing but (with lds) the wave's own
// LDS reads: __syncthreads' release fence would also wait for every copy in
// flight, the next stage's included.
template <bool kLds>
__device__ __forceinline__ void copy_barrier() {
  if (kLds) __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  // s_waitcnt vmcnt(N), the other counters left alone (gfx9 encoding)
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

template <int MT, int SBS>
__global__ __launch_bounds__(256) void gemm_q4k_skinny_dma_kernel(const SkDmaArgs a, int nsb,
                                                                  const int8_t* __restrict__ yq,
                                                                  const float* __restrict__ yd, int M) {
  using D = SkDma<MT, SBS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const bool hin = kq >= 2;
  const int hb = 16 * (kq & 1);
  const uint32_t K = (uint32_t)nsb * 256u;
  const uint32_t rowbytes = (uint32_t)nsb * 144u;

  // the wave's tile: weight t (selects: a dynamic index into the argument
  // arrays would copy them to private memory), its first row there
  const int tile = (int)blockIdx.x * 4 + wv;
  const bool live = tile < a.tile_end[kMaxTargets - 1];
  // (a dead tile of the last workgroup copies rows of the last weight)
  const int t = !live ? a.tg.count - 1
                      : tile < a.tile_end[0] ? 0 : tile < a.tile_end[1] ? 1 : tile < a.tile_end[2] ? 2 : 3;
  auto pick = [&](const auto& arr) { return t == 0 ? arr[0] : t == 1 ? arr[1] : t == 2 ? arr[2] : arr[3]; };
  const int tb = t == 0 ? 0 : t == 1 ? a.tile_end[0] : t == 2 ? a.tile_end[1] : a.tile_end[2];
  const int64_t wbeg = t == 0 ? 0 : t == 1 ? a.tg.row_end[0] : t == 2 ? a.tg.row_end[1] : a.tg.row_end[2];
  const int64_t wrows = pick(a.tg.row_end) - wbeg;
  const int64_t r0 = live ? (int64_t)(tile - tb) * 16 : 0;  // within weight t
  const uint8_t* __restrict__ W = (const uint8_t*)pick(a.tg.w);

  // per-lane copy offsets (fixed over the stages; the stage adds its
  // super-block to the uniform base)
  uint32_t woff[D::kWCopies];
#pragma unroll
  for (int u = 0; u < D::kWCopies; u++) {
    const int sl = 64 * u + lane;
    const int row = sl / D::kWSlots, q = sl - row * D::kWSlots;
    int64_t gr = r0 + (row < 16 ? row : 0);
    gr = gr < wrows ? gr : wrows - 1;
    woff[u] = (uint32_t)gr * rowbytes + 16u * (uint32_t)(q < 9 * SBS ? q : 0);
  }
  uint32_t aoff[D::kACopies];
#pragma unroll
  for (int u = 0; u < D::kACopies; u++) {
    const int sl = 64 * (wv * D::kACopies + u) + lane;
    const int row = sl / D::kASlots, q = sl - row * D::kASlots;
    const int ar = row < D::AR ? (row < M ? row : M - 1) : 0;
    aoff[u] = (uint32_t)ar * K + 16u * (uint32_t)(q < 16 * SBS ? q : 0);
  }
  uint32_t doff;
  {
    const int d = 64 * wv + lane;
    const int row = d / SBS, j = d - row * SBS;
    const int ar = row < D::AR ? (row < M ? row : M - 1) : 0;
    doff = 4u * ((uint32_t)ar * (uint32_t)nsb + (uint32_t)j);
  }
  auto issue = [&](int st, int sb) {
    uint8_t* const base = smem + st * D::kStage;
#pragma unroll
    for (int u = 0; u < D::kWCopies; u++)
      dma16(W + 144 * (int64_t)sb, woff[u], lds_addr(base + wv * D::kWStage + 1024 * u));
#pragma unroll
    for (int u = 0; u < D::kACopies; u++)
      dma16(yq + 256 * (int64_t)sb, aoff[u], lds_addr(base + 4 * D::kWStage + 1024 * (wv * D::kACopies + u)));
    dma4(yd + sb, doff, lds_addr(base + 4 * D::kWStage + D::kAStage + 256 * wv));
  };

  float accD[MT][4], accM[MT][4];
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) accD[m][i] = accM[m][i] = 0.0f;

  // one super-block j of stage st: both passes, the min pass, the f32 epilogue
  // (the register-staged kernel's arithmetic)
  auto compute1 = [&](int st, int j) {
    // each f32 operation rounded on its own (no contraction into fma)
#pragma clang fp contract(off)
    const uint8_t* const base = smem + st * D::kStage;
    const uint8_t* rowp = base + wv * D::kWStage + r16 * (16 * D::kWSlots) + 144 * j;
    const uint4 hdr = *(const uint4*)rowp;
    uint4 code[4];
#pragma unroll
    for (int c = 0; c < 4; c++) code[c] = *(const uint4*)(rowp + 16 + 32 * c + hb);
    i4v am[MT][4];
    float dy[MT][4];
    const uint8_t* const ab = base + 4 * D::kWStage;
    const float* const db = (const float*)(ab + D::kAStage);
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
      for (int c = 0; c < 4; c++)
        am[m][c] = *(const i4v*)(ab + (16 * m + r16) * (16 * D::kASlots) + 256 * j + 64 * c + 16 * kq);
#pragma unroll
      for (int i = 0; i < 4; i++) dy[m][i] = db[(16 * m + 4 * kq + i) * SBS + j];
    }
    // scales and mins (get_scale_min_k4, utils.rs:50-60)
    const uint32_t u0 = hdr.y, u1 = hdr.z, u2 = hdr.w;
    const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
    const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = h2f((uint16_t)(hdr.x & 0xFFFF));
    const float dmin = h2f((uint16_t)(hdr.x >> 16));
    i4v T[MT], Tm[MT];
    const i4v zero = {0, 0, 0, 0};
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int sj = 2 * c + (hin ? 1 : 0);
        const uint32_t scv = ((sj < 4 ? s03 : s47) >> (8 * (sj & 3))) & 0xFF;
        const uint32_t f = sk_dup16(pass == 0 ? scv >> 3 : scv & 7);
        i4v bq;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t w = sk_word(code[c], e);
          bq[e] = (int)sk_pkmul(hin ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu, f);
        }
#pragma unroll
        for (int m = 0; m < MT; m++)
          T[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[m][c], bq, (pass == 0 && c == 0) ? zero : T[m], 0, 0, 0);
      }
      if (pass == 0) {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
          for (int i = 0; i < 4; i++) T[m][i] <<= 3;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int sj = 2 * c + (hin ? 1 : 0);
      const uint32_t mv = ((sj < 4 ? m03 : m47) >> (8 * (sj & 3))) & 0xFF;
      const int mb = (int)(mv * 0x01010101u);
      const i4v bm = {mb, mb, mb, mb};
#pragma unroll
      for (int m = 0; m < MT; m++)
        Tm[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[m][c], bm, c == 0 ? zero : Tm[m], 0, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        accD[m][i] = accD[m][i] + (dw * dy[m][i]) * (float)T[m][i];
        accM[m][i] = accM[m][i] + (dmin * dy[m][i]) * (float)Tm[m][i];
      }
  };

  // every wave issues the same copies every stage (a dead tile's copies read
  // its weight's rows, clamped), so vmcnt counts whole stages
  const int nst = nsb / SBS;
  issue(0, 0);
  if (nst > 1) issue(1, SBS);
  for (int s = 0; s < nst; s++) {
    if (s + 1 < nst)
      wait_vm<D::kCopies>();
    else
      wait_vm<0>();
    copy_barrier<false>();  // every wave's copies of stage s are in LDS
#pragma unroll
    for (int j = 0; j < SBS; j++) compute1(s & 1, j);
    copy_barrier<true>();  // stage s read by every wave before its buffer is refilled
    if (s + 2 < nst) issue(s & 1, (s + 2) * SBS);
  }
  if (!live) return;
  float* const out = pick(a.tg.dst) + r0 + r16;
  const int64_t ldd = pick(a.tg.ldd);
  if (r0 + r16 < wrows) {
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int ar = 16 * m + 4 * kq + i;
        if (ar < M) out[(int64_t)ar * ldd] = __fsub_rn(accD[m][i], accM[m][i]);
      }
  }
}

template <int MT, int SBS>
hipError_t launch_sk_dma(const MvTargets& t, int nsb, const ActPlanes& p, int64_t rows, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  using D = SkDma<MT, SBS>;
  SkDmaArgs a{};
  a.tg = t;
  int tiles = 0;
  for (int i = 0; i < kMaxTargets; i++) {
    if (i < t.count) {
      const int64_t n = t.row_end[i] - (i ? t.row_end[i - 1] : 0);
      tiles += (int)((n + 15) / 16);
    }
    a.tile_end[i] = tiles;
  }
  // unused entries repeat the last weight (no tiles of their own)
  for (int i = t.count; i < kMaxTargets; i++) {
    a.tg.w[i] = t.w[t.count - 1];
    a.tg.dst[i] = t.dst[t.count - 1];
    a.tg.ldd[i] = t.ldd[t.count - 1];
    a.tg.row_end[i] = t.row_end[t.count - 1];
  }
  const size_t lds = 2 * (size_t)D::kStage;
  constexpr auto* kfn = &gemm_q4k_skinny_dma_kernel<MT, SBS>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<dim3((unsigned)((tiles + 3) / 4)), 256, lds, st>>>(a, nsb, p.codes, p.d, (int)rows);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The register-staged kernel's product for narrow weights and up to 16 rows
// with each wave's operands copied straight to LDS: a workgroup owns one
// 16-row tile, its 4 waves split the super-blocks of K as that kernel's do
// and add their partial sums in wave order, and each super-block's
// arithmetic is that kernel's, so a row's bits are the same. A wave copies
// its own super-blocks (the tile's 16 x 144 bytes, MR activation rows and
// their scales) into a ring of NS stages, NS - 1 in flight while it computes
// one, without holding them in registers, so more waves fit a CU. MR (4, 8
// or 16) activation rows are copied, M <= MR; fragment rows past them read
// row MR - 1 and their outputs are never stored. Tiles are numbered weight
// after weight (a ragged last tile reads its weight's last row again).
// ---------------------------------------------------------------------------
template <int MR, int NS>
struct SkKs {
  static constexpr int kWSlots = 10;                           // 16-byte slots a staged weight row (9 + 1: banks)
  static constexpr int kWCopies = (16 * kWSlots + 63) / 64;    // 3
  static constexpr int kASlots = 17;                           // a staged activation row (16 + 1)
  static constexpr int kACopies = (MR * kASlots + 63) / 64;
  static constexpr int kW = kWCopies * 1024;
  static constexpr int kA = kACopies * 1024;
  static constexpr int kStage = kW + kA + 256;                 // + the MR scales (one dword copy)
  static constexpr int kCopies = kWCopies + kACopies + 1;      // copies a stage
  static constexpr int kWave = NS * kStage;
  static_assert(MR <= 64 && (NS - 1) * kCopies <= 63, "vmcnt");
  static_assert(kWave >= 4 * 64 * 4, "the partial sums fit a wave's ring");
};

template <int MR, int NS>
__global__ __launch_bounds__(256) void gemm_q4k_skinny_ks_kernel(const SkDmaArgs a, int nsb,
                                                                 const int8_t* __restrict__ yq,
                                                                 const float* __restrict__ yd, int M) {
  using D = SkKs<MR, NS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const bool hin = kq >= 2;
  const int hb = 16 * (kq & 1);
  const uint32_t K = (uint32_t)nsb * 256u;
  const uint32_t rowbytes = (uint32_t)nsb * 144u;
  uint8_t* const ring = smem + wv * D::kWave;

  // the workgroup's tile: weight t (by selects), its first row there
  const int tile = (int)blockIdx.x;
  const int t = tile < a.tile_end[0] ? 0 : tile < a.tile_end[1] ? 1 : tile < a.tile_end[2] ? 2 : 3;
  auto pick = [&](const auto& arr) { return t == 0 ? arr[0] : t == 1 ? arr[1] : t == 2 ? arr[2] : arr[3]; };
  const int tb = t == 0 ? 0 : t == 1 ? a.tile_end[0] : t == 2 ? a.tile_end[1] : a.tile_end[2];
  const int64_t wbeg = t == 0 ? 0 : t == 1 ? a.tg.row_end[0] : t == 2 ? a.tg.row_end[1] : a.tg.row_end[2];
  const int64_t wrows = pick(a.tg.row_end) - wbeg;
  const int64_t r0 = (int64_t)(tile - tb) * 16;
  const uint8_t* __restrict__ W = (const uint8_t*)pick(a.tg.w);

  // the wave's super-blocks (the register-staged kernel's split)
  const int per = (nsb + 3) / 4;
  const int sb0 = wv * per;
  const int sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  const int len = sb1 > sb0 ? sb1 - sb0 : 0;

  uint32_t woff[D::kWCopies];
#pragma unroll
  for (int u = 0; u < D::kWCopies; u++) {
    const int sl = 64 * u + lane;
    const int row = sl / D::kWSlots, q = sl - row * D::kWSlots;
    int64_t gr = r0 + (row < 16 ? row : 0);
    gr = gr < wrows ? gr : wrows - 1;
    woff[u] = (uint32_t)gr * rowbytes + 16u * (uint32_t)(q < 9 ? q : 0);
  }
  uint32_t aoff[D::kACopies];
#pragma unroll
  for (int u = 0; u < D::kACopies; u++) {
    const int sl = 64 * u + lane;
    const int row = sl / D::kASlots, q = sl - row * D::kASlots;
    const int ar = row < MR ? (row < M ? row : M - 1) : 0;
    aoff[u] = (uint32_t)ar * K + 16u * (uint32_t)(q < 16 ? q : 0);
  }
  const uint32_t doff = 4u * (uint32_t)(lane < MR ? (lane < M ? lane : M - 1) : 0) * (uint32_t)nsb;
  // stage s (super-block sb0 + s, clamped into the wave's range: past it the
  // copies repeat its last super-block, so every step issues the same copies)
  auto issue = [&](int s) {
    const int sb = len == 0 ? 0 : (s < len ? sb0 + s : sb1 - 1);
    uint8_t* const base = ring + (s % NS) * D::kStage;
#pragma unroll
    for (int u = 0; u < D::kWCopies; u++) dma16(W + 144 * (int64_t)sb, woff[u], lds_addr(base + 1024 * u));
#pragma unroll
    for (int u = 0; u < D::kACopies; u++) dma16(yq + 256 * (int64_t)sb, aoff[u], lds_addr(base + D::kW + 1024 * u));
    dma4(yd + sb, doff, lds_addr(base + D::kW + D::kA));
  };

  float accD[4], accM[4];
#pragma unroll
  for (int i = 0; i < 4; i++) accD[i] = accM[i] = 0.0f;
  const int arow = r16 < MR ? r16 : MR - 1;
  auto compute = [&](int s) {
    // each f32 operation rounded on its own (no contraction into fma)
#pragma clang fp contract(off)
    const uint8_t* const base = ring + (s % NS) * D::kStage;
    const uint8_t* rowp = base + r16 * (16 * D::kWSlots);
    const uint4 hdr = *(const uint4*)rowp;
    uint4 code[4];
#pragma unroll
    for (int c = 0; c < 4; c++) code[c] = *(const uint4*)(rowp + 16 + 32 * c + hb);
    i4v am[4];
    float dy[4];
#pragma unroll
    for (int c = 0; c < 4; c++) am[c] = *(const i4v*)(base + D::kW + arow * (16 * D::kASlots) + 64 * c + 16 * kq);
    const float* const db = (const float*)(base + D::kW + D::kA);
#pragma unroll
    for (int i = 0; i < 4; i++) dy[i] = db[4 * kq + i < MR ? 4 * kq + i : MR - 1];
    // scales and mins (get_scale_min_k4, utils.rs:50-60)
    const uint32_t u0 = hdr.y, u1 = hdr.z, u2 = hdr.w;
    const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
    const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = h2f((uint16_t)(hdr.x & 0xFFFF));
    const float dmin = h2f((uint16_t)(hdr.x >> 16));
    i4v T, Tm;
    const i4v zero = {0, 0, 0, 0};
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int sj = 2 * c + (hin ? 1 : 0);
        const uint32_t scv = ((sj < 4 ? s03 : s47) >> (8 * (sj & 3))) & 0xFF;
        const uint32_t f = sk_dup16(pass == 0 ? scv >> 3 : scv & 7);
        i4v bq;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t w = sk_word(code[c], e);
          bq[e] = (int)sk_pkmul(hin ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu, f);
        }
        T = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[c], bq, (pass == 0 && c == 0) ? zero : T, 0, 0, 0);
      }
      if (pass == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) T[i] <<= 3;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int sj = 2 * c + (hin ? 1 : 0);
      const uint32_t mv = ((sj < 4 ? m03 : m47) >> (8 * (sj & 3))) & 0xFF;
      const int mb = (int)(mv * 0x01010101u);
      const i4v bm = {mb, mb, mb, mb};
      Tm = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[c], bm, c == 0 ? zero : Tm, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      accD[i] = accD[i] + (dw * dy[i]) * (float)T[i];
      accM[i] = accM[i] + (dmin * dy[i]) * (float)Tm[i];
    }
  };

  // The ring: stages 0 .. NS - 2 in flight before the loop; step s issues
  // stage s + NS - 1 into the buffer stage s - 1 used (read by now), waits
  // for stage s (the NS - 1 stages issued after it may stay in flight) and
  // computes it.
#pragma unroll
  for (int s = 0; s < NS - 1; s++) issue(s);
  for (int s = 0; s < len; s++) {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0): stage s - 1's reads done
    asm volatile("" ::: "memory");
    issue(s + NS - 1);
    wait_vm<(NS - 1) * D::kCopies>();
    asm volatile("" ::: "memory");
    compute(s);
  }
  // every copy landed before the ring holds the partial sums
  wait_vm<0>();
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  asm volatile("" ::: "memory");
  float* const part = (float*)ring;
#pragma unroll
  for (int i = 0; i < 4; i++) part[i * 64 + lane] = __fsub_rn(accD[i], accM[i]);
  __syncthreads();
  if (wv == 0 && r0 + r16 < wrows) {
    float* const out = pick(a.tg.dst) + r0 + r16;
    const int64_t ldd = pick(a.tg.ldd);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v = ((const float*)smem)[i * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; w++) v = __fadd_rn(v, ((const float*)(smem + w * D::kWave))[i * 64 + lane]);
      const int ar = 4 * kq + i;
      if (ar < M) out[(int64_t)ar * ldd] = v;
    }
  }
}

template <int MR, int NS>
hipError_t launch_sk_ks(const MvTargets& t, int nsb, const ActPlanes& p, int64_t rows, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  using D = SkKs<MR, NS>;
  SkDmaArgs a{};
  a.tg = t;
  int tiles = 0;
  for (int i = 0; i < kMaxTargets; i++) {
    if (i < t.count) {
      const int64_t n = t.row_end[i] - (i ? t.row_end[i - 1] : 0);
      tiles += (int)((n + 15) / 16);
    }
    a.tile_end[i] = tiles;
  }
  for (int i = t.count; i < kMaxTargets; i++) {
    a.tg.w[i] = t.w[t.count - 1];
    a.tg.dst[i] = t.dst[t.count - 1];
    a.tg.ldd[i] = t.ldd[t.count - 1];
    a.tg.row_end[i] = t.row_end[t.count - 1];
  }
  const size_t lds = 4 * (size_t)D::kWave;
  constexpr auto* kfn = &gemm_q4k_skinny_ks_kernel<MR, NS>;
  if (lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<dim3((unsigned)tiles), 256, lds, st>>>(a, nsb, p.codes, p.d, (int)rows);
  return hipGetLastError();
}

}  // namespace

int gemm_q4k_skinny_max_rows() { return 32; }

bool gemm_q4k_skinny_fits(int64_t k, int64_t rows) {
  return k % 256 == 0 && rows >= 1 && rows <= 32;
}

// the register-staged kernel (one or two 16-row tiles a workgroup, the
// super-blocks split over 4 waves)
static hipError_t launch_gemm_q4k_skinny_reg(const MvTargets& t, int nsb, const ActPlanes& p, int64_t rows, int cus,
                                             hipStream_t st) {
  // two 16-row tiles a workgroup where the rows fill the CUs twice over
  const int64_t n_total = t.row_end[t.count - 1];
  const bool wide = n_total >= (int64_t)cus * 32 * 2;
  // narrow weights of up to 16 rows: the same product with copies to LDS
  // (weights under 4 GiB: its lanes form weight offsets in 32 bits)
  bool small = !wide && rows <= 16;
  for (int i = 0; i < t.count && small; i++)
    small = (t.row_end[i] - (i ? t.row_end[i - 1] : 0)) * nsb * 144 < ((int64_t)1 << 32);
  // (two stages a wave: three workgroups a CU at 8 rows; C5 at 8 / 16 rows
  // 6.51 / 7.20 -> 6.39 / 7.02 ms a forward, three stages 6.43 / 7.21)
  if (small) {
    if (rows <= 4) return launch_sk_ks<4, 2>(t, nsb, p, rows, st);
    if (rows <= 8) return launch_sk_ks<8, 2>(t, nsb, p, rows, st);
    return launch_sk_ks<16, 2>(t, nsb, p, rows, st);
  }
  if (rows <= 16) return wide ? launch_sk<1, 2, 4>(t, nsb, p, rows, st) : launch_sk<1, 1, 4>(t, nsb, p, rows, st);
  return wide ? launch_sk<2, 2, 4>(t, nsb, p, rows, st) : launch_sk<2, 1, 4>(t, nsb, p, rows, st);
}

hipError_t launch_gemm_q4k_skinny(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, int cus,
                                  hipStream_t st) {
  const int nsb = (int)(k / 256);
  // weights of at least 64 rows a CU (C5's gate and up) take the
  // copy-staged kernel, two super-blocks a stage (C5 at 8 / 16 rows: 6.75 /
  // 7.68 -> 6.68 / 7.30 ms a forward; four a stage hold 122 KiB of LDS, one
  // workgroup a CU, 7.51 / 8.19; one a stage 6.75 / 7.41); the choice is each
  // weight's own, so a weight's bits do not depend on the weights it shares
  // a launch with. Its lanes form weight offsets in 32 bits, so a weight of
  // 4 GiB or more stays on the register-staged kernel (64-bit addressing).
  constexpr int kDmaSbs = 2;
  MvTargets wide{}, narrow{};
  if (rows <= 16 && nsb % kDmaSbs == 0) {
    int64_t prev = 0, we = 0, ne = 0;
    for (int i = 0; i < t.count; i++) {
      const int64_t n = t.row_end[i] - prev;
      prev = t.row_end[i];
      const bool to_dma = n >= (int64_t)64 * cus && n * nsb * 144 < ((int64_t)1 << 32);
      MvTargets& g = to_dma ? wide : narrow;
      int64_t& e = to_dma ? we : ne;
      e += n;
      g.w[g.count] = t.w[i];
      g.dst[g.count] = t.dst[i];
      g.ldd[g.count] = t.ldd[i];
      g.row_end[g.count] = e;
      g.count++;
    }
    if (wide.count > 0) {
      const hipError_t e1 = launch_sk_dma<1, kDmaSbs>(wide, nsb, p, rows, st);
      if (e1 != hipSuccess || narrow.count == 0) return e1;
      return launch_gemm_q4k_skinny_reg(narrow, nsb, p, rows, cus, st);
    }
  }
  return launch_gemm_q4k_skinny_reg(t, nsb, p, rows, cus, st);
}

}  // namespace qmm
