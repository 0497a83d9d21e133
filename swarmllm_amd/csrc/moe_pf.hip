// moe_pf.hip — grouped expert products of prompt-size routings on the f16 /
// bf16 matrix cores of gfx950: the work of candle-kernels'
// moe_gemm_gguf_prefill (vendor/candle/candle-kernels/src/moe/
// moe_wmma_gguf.cu:191-371, launched at :450-535), which
// src/inference/layers/moe_card.rs:48-170 calls for a chunk of more than
// MOE_CARD_ONE_ROW_MAX_TOKENS = 8 tokens (src/inference/layers/mod.rs:475,
// 2753).
//
// Numerics are the reference's: each weight value is dequantized in f32 as
// to_float computes it and rounded to the input's 16-bit type (f16 or bf16,
// to nearest even); the input is in that type; the products are summed in f32
// by the matrix cores; dst[p][j] = scale_p * sum. The routing (entries, runs,
// per-pair or per-token input rows, routing weights, out-of-range entries
// writing nothing) is that of the grouped decode product (moe.hip).
//
// Shape of the work: the routing's runs (moe_runs.h) are cut into chunks of
// up to 64 entries of one expert, in a table written by the one-workgroup
// prologue launch (moe_pf_prep_kernel). A workgroup of 4 waves takes a chunk
// and a tile of 128 weight rows of the chunk's expert and walks k in stages of
// 128 values. For each stage, direct global-to-LDS copies bring each weight
// row's bytes of the stage (the 16-byte aligned windows of the byte ranges the
// stage reads) and the chunk's input rows (128 values each, 16-byte pieces
// XOR-swizzled by row) into one half of double buffers while the waves work on
// the other half; two workgroups share a CU, one computing while the other
// waits for its copies. Each wave owns 32 weight rows: lane L dequantizes row
// L%32 into the B operand of v_mfma_f32_32x32x16_{f16,bf16}, which it applies
// to the chunk's first and (past 32 entries) second 32 entries, 8 steps a
// stage. The order in which a stage's 128 values enter the steps is chosen per
// format so that a lane's 8 values of a step come from 8 consecutive bytes of
// its row; the A side reads the input values of the same positions, and any
// order gives the same sum of products.
#include "b32_common.h"
#include "lds_copy.h"
#include "moe_runs.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef _Float16 pf_h8 __attribute__((ext_vector_type(8)));
typedef __bf16 pf_b8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_h2 __attribute__((ext_vector_type(2)));
typedef __bf16 pf_b2 __attribute__((ext_vector_type(2)));
typedef float pf_f2 __attribute__((ext_vector_type(2)));
typedef float pf_f16 __attribute__((ext_vector_type(16)));
typedef unsigned pf_u4 __attribute__((ext_vector_type(4)));

constexpr int kPfM = 64;                   // routing entries a chunk: two MFMA row tiles
constexpr int kPfK = 128;                  // values a stage
constexpr int kPfRowBytes = kPfK * 2;      // an input row's stage (16-bit values)
constexpr int kPfABytes = kPfM * kPfRowBytes;
constexpr int kPfACopies = kPfABytes / 1024;
constexpr int kPfW = 4;                    // waves a workgroup
constexpr int kPfNT = 32 * kPfW;           // weight rows a workgroup
constexpr int kPfPrepThreads = 256;

// A weight row's stage: the byte ranges it reads (up to 3 regions, each an
// offset from the stage's base and a length, with their change from the first
// half of a super-block to the second: K-quant stages are half super-blocks),
// the 16-byte pieces of each region's aligned window, and the LDS row stride
// in pieces (odd, so the 32 rows a wave reads in one instruction fall on
// distinct banks).
//   Q4_K (16-byte aligned rows): d, dmin, scales (16 bytes); qs[64h .. +63].
//   Q6_K: ql[64h .. +63]; qh[32h .. +31]; sc[8h ..] and d (bytes 192 + 8h to
//         209).
//   32-value formats: 4 blocks.
template <int FMT>
struct PfShape {
  static constexpr bool KQ = FMT == T_Q4_K || FMT == T_Q6_K;
  static constexpr int BB = FMT == T_Q4_K ? 144 : FMT == T_Q6_K ? 210 : FMT == T_Q8_0 ? 34 : FMT == T_IQ4_NL ? 18 : 17;
  static constexpr int NR = FMT == T_Q4_K ? 2 : FMT == T_Q6_K ? 3 : 1;
  __host__ __device__ static constexpr int off0(int r) {
    return FMT == T_Q4_K ? (r == 0 ? 0 : 16) : FMT == T_Q6_K ? (r == 0 ? 0 : r == 1 ? 128 : 192) : 0;
  }
  __host__ __device__ static constexpr int dlt(int r) {
    return FMT == T_Q4_K ? (r == 0 ? 0 : 64) : FMT == T_Q6_K ? (r == 0 ? 64 : r == 1 ? 32 : 8) : 0;
  }
  __host__ __device__ static constexpr int len0(int r) {
    return FMT == T_Q4_K ? (r == 0 ? 16 : 64) : FMT == T_Q6_K ? (r == 0 ? 64 : r == 1 ? 32 : 18) : 4 * BB;
  }
  __host__ __device__ static constexpr int dlen(int r) { return FMT == T_Q6_K && r == 2 ? -8 : 0; }
  __host__ __device__ static constexpr int pieces(int r) {
    return FMT == T_Q4_K ? len0(r) / 16 : (len0(r) + 30) / 16;
  }
  static constexpr int P = pieces(0) + (NR > 1 ? pieces(1) : 0) + (NR > 2 ? pieces(2) : 0);
  static constexpr int Ps = P | 1;
  static constexpr int WCopies = (kPfNT * Ps + 63) / 64;
  static constexpr int WBytes = WCopies * 1024;
  static constexpr int Copies = WCopies + kPfACopies;
  static constexpr int CopiesPerWave = (Copies + kPfW - 1) / kPfW;
  static constexpr int Lds = 2 * kPfABytes + 2 * WBytes + 3 * kPfM * 4;
  static_assert(Lds <= 80 * 1024, "two workgroups' buffers fit a CU's LDS");
};

// Two f32 values rounded to the 16-bit type (to nearest even), packed.
template <bool BF>
__device__ __forceinline__ uint32_t pk2(float a, float b) {
  const pf_f2 v = {a, b};
  if constexpr (BF)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pf_b2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pf_h2));
}

template <bool BF>
__device__ __forceinline__ pf_f16 mfma16(pf_u4 a, pf_u4 b, pf_f16 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(pf_b8, a), __builtin_bit_cast(pf_b8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(pf_h8, a), __builtin_bit_cast(pf_h8, b), c, 0, 0,
                                                  0);
}

// The 8 byte values of w0, w1 (byte i of w0 first) through fma(d, byte, c),
// packed as the B operand's 8 16-bit values. Every caller's d * byte is exact
// in f32, so the result is the single rounding of d * byte + c that to_float's
// multiply-then-add gives.
template <bool BF>
__device__ __forceinline__ pf_u4 deq8(uint32_t w0, uint32_t w1, float d, float c) {
  // opaque to the compiler, so that byte i converts in one v_cvt_f32_ubyte<i>
  // rather than a bit-field extract of the caller's mask and a conversion
  asm("" : "+v"(w0), "+v"(w1));
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    v[i] = __builtin_fmaf(d, (float)((w0 >> (8 * i)) & 0xFF), c);
    v[4 + i] = __builtin_fmaf(d, (float)((w1 >> (8 * i)) & 0xFF), c);
  }
  pf_u4 r;
  r.x = pk2<BF>(v[0], v[1]);
  r.y = pk2<BF>(v[2], v[3]);
  r.z = pk2<BF>(v[4], v[5]);
  r.w = pk2<BF>(v[6], v[7]);
  return r;
}

// One stage of a weight row for lane half h from its LDS window `win`; `o`
// is the stage base's offset in its 16-byte piece, `hf` the super-block half
// (K-quants), nb_left the row's 32-value blocks from this stage on (blocks
// past the row are skipped). step(piece, b) for each of the 8 steps, `piece`
// the 8-value group (of the stage's 16) whose values b holds.
template <int FMT, bool BF, class Step>
__device__ __forceinline__ void pf_stage(const uint8_t* win, int o, int hf, int h, int nb_left, uint32_t t0,
                                         uint32_t t1, uint32_t t2, uint32_t t3, Step&& step) {
  if constexpr (FMT == T_Q4_K) {
    // d, dmin, 12 scale bytes, then qs[128]: value 64p + l is the low nibble
    // of qs[32p + l], value 64p + 32 + l its high nibble (l < 32); sub-block
    // j = 2p (low) and 2p + 1 (high) scale d * sc_j, offset dmin * m_j
    // (k_quants.rs to_float of BlockQ4K). This half holds p = 2 hf, 2 hf + 1.
    // Lane half h takes bytes 32p + 16h .. +15: steps t = 0, 1 the low
    // nibbles of its bytes 0-7, 8-15, t = 2, 3 the high nibbles.
    const uint4 hv = *(const uint4*)win;
    const uint32_t hd[4] = {hv.x, hv.y, hv.z, hv.w};
    const float d = h2f((uint16_t)(hd[0] & 0xFFFF)), dm = h2f((uint16_t)(hd[0] >> 16));
    auto sb = [&](int i) { return (int)((hd[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF); };
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
      int sc[2], mn[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int j = 4 * hf + 2 * pp + u;  // uniform
        if (j < 4) {
          sc[u] = sb(j) & 63;
          mn[u] = sb(j + 4) & 63;
        } else {
          sc[u] = (sb(j + 4) & 0xF) | ((sb(j - 4) >> 6) << 4);
          mn[u] = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
        }
      }
      const float d1a = d * (float)sc[0], m1a = dm * (float)mn[0];
      // the high nibbles are read in place (16 q): the scale / 16 is exact
      const float d1b = d * (float)sc[1] * 0.0625f, m1b = dm * (float)mn[1];
      const uint4 qv = *(const uint4*)(win + 16 + 32 * pp + 16 * h);
      step(8 * pp + 2 * h, deq8<BF>(qv.x & 0x0F0F0F0Fu, qv.y & 0x0F0F0F0Fu, d1a, -m1a));
      step(8 * pp + 2 * h + 1, deq8<BF>(qv.z & 0x0F0F0F0Fu, qv.w & 0x0F0F0F0Fu, d1a, -m1a));
      step(8 * pp + 4 + 2 * h, deq8<BF>(qv.x & 0xF0F0F0F0u, qv.y & 0xF0F0F0F0u, d1b, -m1b));
      step(8 * pp + 4 + 2 * h + 1, deq8<BF>(qv.z & 0xF0F0F0F0u, qv.w & 0xF0F0F0F0u, d1b, -m1b));
    }
  } else if constexpr (FMT == T_Q6_K) {
    // ql[128], qh[64], sc[16] (int8), d: in half g (values 128g ..), value
    // 128g + 32j + l (l < 32) is the 6-bit code of ql[64g + 32(j&1) + l]'s
    // low (j < 2) or high nibble and bits 2j, 2j+1 of qh[32g + l], minus 32,
    // times d * sc[8g + l/16 + 2j] (to_float of BlockQ6K). This half g = hf;
    // its regions: ql[64g ..] at window byte o, qh[32g ..] at 80 + o, sc[8g ..]
    // then d at 128 + ((o + 8g) & 15). Lane half h takes l = 16u + 8h .. +7.
    const int o2 = 128 + ((o + 8 * hf) & 15);
    uint32_t scw[2];
    lds_words<2>(win, o2, scw);
    const float d = h2f((uint16_t)lds_u16(win, o2 + 16 - 8 * hf));
#pragma unroll
    for (int u = 0; u < 2; u++) {
      uint32_t A[2], B[2], H[2];
      lds_words<2>(win, o + 16 * u + 8 * h, A);
      lds_words<2>(win, o + 32 + 16 * u + 8 * h, B);
      lds_words<2>(win, 80 + o + 16 * u + 8 * h, H);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t* src = (j & 1) ? B : A;
        uint32_t c[2];
#pragma unroll
        for (int w = 0; w < 2; w++) {
          const uint32_t nib = (j & 2) ? ((src[w] >> 4) & 0x0F0F0F0Fu) : (src[w] & 0x0F0F0F0Fu);
          c[w] = nib | (((H[w] >> (2 * j)) & 0x03030303u) << 4);
        }
        const int si = u + 2 * j;
        const float ds = d * (float)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFF);
        // ds (code - 32) as one rounding of ds * code - 32 ds
        step(4 * j + 2 * u + h, deq8<BF>(c[0], c[1], ds, -32.0f * ds));
      }
    }
  } else {
    // 4 blocks of 32 values. Q8_0: f16 d, 32 int8 codes; lane half h takes
    // codes 16t + 8h .. +7 for steps t = 0, 1. IQ4_NL (f16 d) and MXFP4 (e8m0
    // scale, halved against the doubled table): value l < 16 the low nibble of
    // qs[l], 16 + l the high; lane half h takes qs[8h .. 8h+7], the low
    // nibbles at t = 0, the high at t = 1. Signed codes are read as
    // unsigned (code + 128) and fma(d, code + 128, -128 d): exact.
    constexpr int B = PfShape<FMT>::BB;
    constexpr int Head = FMT == T_MXFP4 ? 1 : 2;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      if (b >= nb_left) break;  // uniform
      const int ob = o + B * b;
      float d;
      if constexpr (FMT == T_MXFP4)
        d = e8m0_half(lds_u32(win, ob) & 0xFF);
      else
        d = h2f((uint16_t)lds_u16(win, ob));
      if constexpr (FMT == T_Q8_0) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
          uint32_t q[2];
          lds_words<2>(win, ob + 2 + 16 * t + 8 * h, q);
          step(4 * b + 2 * t + h, deq8<BF>(q[0] ^ 0x80808080u, q[1] ^ 0x80808080u, d, -128.0f * d));
        }
      } else {
        uint32_t q[2];
        lds_words<2>(win, ob + Head + 8 * h, q);
        pf_u4 bv[2];
        bool table = true;
        if constexpr (FMT == T_MXFP4) {
          // E2M1 codes times the scale 2^(e-127), rounded to the 16-bit type,
          // by the converter of gfx950 (two codes of a byte a conversion, its
          // low nibble first): the table path's value bit for bit (checked on
          // every code at every scale byte but 255, whose 2^128 is not an f32;
          // and the sign of a zero code, invisible in any sum of products).
          // Pairs of the lane's bytes' low (t = 0) or high nibbles are packed
          // into one byte each, bytes 0 and 2 of a word.
          const uint32_t e = lds_u32(win, ob) & 0xFF;
          table = e == 255;
          if (!table) {
            const float sc = __builtin_bit_cast(float, e == 0 ? 0x00400000u : e << 23);
#pragma unroll
            for (int t = 0; t < 2; t++) {
              uint32_t r[4];
#pragma unroll
              for (int w = 0; w < 2; w++) {
                uint32_t v = t ? (q[w] >> 4) & 0x0F0F0F0Fu : q[w] & 0x0F0F0F0Fu;
                v |= v >> 4;
                if constexpr (BF) {
                  r[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 0));
                  r[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 2));
                } else {
                  r[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 0));
                  r[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 2));
                }
              }
              bv[t].x = r[0];
              bv[t].y = r[1];
              bv[t].z = r[2];
              bv[t].w = r[3];
            }
          }
        }
        if (table) {
#pragma unroll
          for (int t = 0; t < 2; t++) {
            const uint32_t c0 = (uint32_t)lut16_at(q[0], t ? 4 : 0, t0, t1, t2, t3);
            const uint32_t c1 = (uint32_t)lut16_at(q[1], t ? 4 : 0, t0, t1, t2, t3);
            bv[t] = deq8<BF>(c0 ^ 0x80808080u, c1 ^ 0x80808080u, d, -128.0f * d);
          }
        }
        step(4 * b + h, bv[0]);
        step(4 * b + 2 + h, bv[1]);
      }
    }
  }
}

template <int FMT, bool BF>
__global__ __launch_bounds__(64 * kPfW, 2) void moe_pf_kernel(
    const uint8_t* __restrict__ W, int64_t n, int64_t k, int64_t rb, int64_t estride, int num_experts,
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ chunks,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m, float* __restrict__ dst,
    int64_t ldd) {
  using S = PfShape<FMT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const sA = smem;                          // [2][64 rows][256 B]
  uint8_t* const sW = smem + 2 * kPfABytes;          // [2][WBytes]
  int* const s_in = (int*)(sW + 2 * S::WBytes);      // the chunk's input rows
  int* const s_out = s_in + kPfM;                    // output rows (-1: none)
  float* const s_sc = (float*)(s_out + kPfM);        // routing weights

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * kPfNT;
  const int nb32 = (int)(k / 32);
  const int nst = (int)((k + kPfK - 1) / kPfK);
  const int nch = __builtin_amdgcn_readfirstlane(chunks[0]);
  uint32_t t0 = 0, t1 = 0, t2 = 0, t3 = 0;
  if constexpr (FMT == T_IQ4_NL || FMT == T_MXFP4) {
    const Lut32<FMT> lut;
    t0 = lut.t0;
    t1 = lut.t1;
    t2 = lut.t2;
    t3 = lut.t3;
  }
  // this lane's weight row (rows past n read the last; never stored)
  const int64_t wrow = n0 + 32 * wv + r32 < n ? n0 + 32 * wv + r32 : n - 1;
  const uint32_t wrow_off = (uint32_t)(wrow * rb);
  // a stage's base in a weight row: its super-block (K-quants) or 4 blocks
  auto stage_base = [&](int st) -> uint32_t {
    return S::KQ ? (uint32_t)(S::BB * (st >> 1)) : (uint32_t)(4 * S::BB * st);
  };

  for (int c = blockIdx.y; c < nch; c += gridDim.y) {
    const int start = __builtin_amdgcn_readfirstlane(chunks[1 + 3 * c]);
    const int cnt = __builtin_amdgcn_readfirstlane(chunks[2 + 3 * c]);
    const int e = __builtin_amdgcn_readfirstlane(chunks[3 + 3 * c]);
    if (e < 0 || e >= num_experts) continue;  // uniform: the entries write nothing
    if (tid < kPfM) {
      const int p = tid < cnt ? ids[start + tid] : -1;
      const bool ok = p >= 0 && p < size_m;
      s_in[tid] = ok ? (topk_w ? p : p / topk) : 0;
      s_out[tid] = ok ? p : -1;
      s_sc[tid] = ok && topk_w ? topk_w[p] : 1.0f;
    }
    __syncthreads();
    const uint8_t* const We = W + (int64_t)e * estride;
    const bool two = cnt > 32;  // the second row tile has entries

    // The copies of a stage into buffer half `buf`. Weight copy i moves window
    // pieces f = 64 i + L: row f / Ps, piece f % Ps, which is piece q of region
    // r's aligned window (clamped to the piece holding the region's last byte
    // in the row). Input copy i moves rows 4i .. 4i + 3: lane L writes position
    // L % 16 of row m = 4i + L/16, which holds piece (L % 16) ^ (m % 16) of the
    // row's stage (clamped to the row's last piece); copies of rows past the
    // chunk's entries are skipped. The waves take copies wv, wv + W, ...; a
    // lane keeps, per copy, its row's byte offset and its piece's offset in the
    // window (with the region number in the high half).
    uint32_t c_row[S::CopiesPerWave], c_pr[S::CopiesPerWave];
#pragma unroll
    for (int u = 0; u < S::CopiesPerWave; u++) {
      const int j = wv + kPfW * u;
      if (j < S::WCopies) {
        const uint32_t f = 64u * (uint32_t)j + (uint32_t)lane;
        const uint32_t r = f / (uint32_t)S::Ps < (uint32_t)kPfNT ? f / (uint32_t)S::Ps : kPfNT - 1;
        const int64_t gr = n0 + r < n ? n0 + r : n - 1;
        int pc = (int)(f % (uint32_t)S::Ps), reg = 0;
        pc = pc < S::P ? pc : S::P - 1;  // the odd stride's spare piece repeats the last
#pragma unroll
        for (int q = 0; q < S::NR - 1; q++)
          if (pc >= S::pieces(reg)) {
            pc -= S::pieces(reg);
            reg++;
          }
        c_row[u] = (uint32_t)(gr * rb);
        c_pr[u] = 16u * (uint32_t)pc | ((uint32_t)reg << 16);
      } else {
        const int m = 4 * (j - S::WCopies) + (lane >> 4);
        c_row[u] = 2u * (uint32_t)s_in[m < kPfM ? m : 0] * (uint32_t)x_stride;
        c_pr[u] = 16u * (uint32_t)((lane & 15) ^ (m & 15));
      }
    }
    auto issue = [&](int st, int buf) {
      const uint32_t sbase = stage_base(st);
      const int hf = st & 1;
      // the regions' offsets from the row and lengths at this stage (uniform)
      uint32_t ra[3], rl[3];
#pragma unroll
      for (int r = 0; r < 3; r++) {
        ra[r] = sbase + (uint32_t)(S::off0(r) + hf * S::dlt(r));
        rl[r] = (uint32_t)(S::len0(r) + hf * S::dlen(r));
      }
#pragma unroll
      for (int u = 0; u < S::CopiesPerWave; u++) {
        const int j = wv + kPfW * u;
        if (j < S::WCopies) {
          const uint32_t reg = c_pr[u] >> 16;
          const uint32_t ro = S::NR == 1 ? ra[0] : reg == 0 ? ra[0] : (S::NR == 2 || reg == 1) ? ra[1] : ra[2];
          const uint32_t rlen = S::NR == 1 ? rl[0] : reg == 0 ? rl[0] : (S::NR == 2 || reg == 1) ? rl[1] : rl[2];
          const uint32_t a = c_row[u] + ro;
          const uint32_t rend = a + rlen, row_end = c_row[u] + (uint32_t)rb;
          const uint32_t send = rend < row_end ? rend : row_end;
          const uint32_t last = (send - 1u) & ~15u, o = (a & ~15u) + (c_pr[u] & 0xFFFFu);
          dma16(We, o < last ? o : last, __builtin_amdgcn_readfirstlane(lds_addr(sW + buf * S::WBytes + 1024 * j)));
        } else if (j < S::Copies && 4 * (j - S::WCopies) < cnt) {
          const uint32_t el = (uint32_t)(kPfRowBytes * st) + c_pr[u];
          const uint32_t lim = 2u * ((uint32_t)k - 8u);
          dma16(x, c_row[u] + (el < lim ? el : lim),
                __builtin_amdgcn_readfirstlane(lds_addr(sA + buf * kPfABytes + 1024 * (j - S::WCopies))));
        }
      }
    };

    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    pf_f16 acc0, acc1;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      acc0[i] = 0.0f;
      acc1[i] = 0.0f;
    }
    const int sw = r32 & 15;  // this lane's A rows' swizzle (rows r32 and 32 + r32)
    for (int st = 0; st < nst; st++) {
      const int cur = st & 1;
      if (st + 1 < nst) issue(st + 1, cur ^ 1);
      const uint8_t* win = sW + cur * S::WBytes + (32 * wv + r32) * (S::Ps * 16);
      const int o = (int)((wrow_off + stage_base(st)) & 15u);
      const uint8_t* arow = sA + cur * kPfABytes + r32 * kPfRowBytes;
      pf_stage<FMT, BF>(win, o, st & 1, h, nb32 - 4 * st, t0, t1, t2, t3, [&](int piece, pf_u4 b) {
        const int ap = 16 * (piece ^ sw);
        acc0 = mfma16<BF>(*(const pf_u4*)(arow + ap), b, acc0);
        if (two) acc1 = mfma16<BF>(*(const pf_u4*)(arow + 32 * kPfRowBytes + ap), b, acc1);
      });
      // the next stage has landed, and every wave is done with this one
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    // lane L holds entries m = 8 (i/4) + 4 h + i%4 (and 32 + m) of weight row r32
    const int64_t col = n0 + 32 * wv + r32;
    if (col < n) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int m = 8 * (i >> 2) + 4 * h + (i & 3);
        const int p = s_out[m];
        if (p >= 0) dst[(int64_t)p * ldd + col] = __fmul_rn(acc0[i], s_sc[m]);
        if (two) {
          const int p1 = s_out[32 + m];
          if (p1 >= 0) dst[(int64_t)p1 * ldd + col] = __fmul_rn(acc1[i], s_sc[32 + m]);
        }
      }
    }
    __syncthreads();  // the entry tables are rewritten by the next chunk
  }
}

// Block 0: the run table and the chunk table of 64 entries. Blocks 1..: the
// input rows into 16-bit values (f32 rounded to nearest even, or a 16-bit
// input copied) at xo [rows][k], 16-byte aligned, 8 values a thread.
template <int XK>
__global__ __launch_bounds__(kPfPrepThreads) void moe_pf_prep_kernel(const int32_t* __restrict__ expert_ids,
                                                                     int size_m, int32_t* __restrict__ runs,
                                                                     int32_t* __restrict__ chunks,
                                                                     const void* __restrict__ x, int64_t x_stride,
                                                                     int64_t k, int64_t rows,
                                                                     uint16_t* __restrict__ xo) {
  if (blockIdx.x == 0) {
    moe_runs_block<kPfPrepThreads>(expert_ids, size_m, runs);
    moe_chunks_block<kPfPrepThreads>(runs, kPfM, chunks);
    return;
  }
  const int64_t groups = rows * (k / 8);
  for (int64_t g = (int64_t)(blockIdx.x - 1) * kPfPrepThreads + threadIdx.x; g < groups;
       g += (int64_t)(gridDim.x - 1) * kPfPrepThreads) {
    const int64_t r = g / (k / 8), c = 8 * (g % (k / 8));
    uint32_t o[4];
    if constexpr (XK == 2) {
      const float* s = (const float*)x + r * x_stride + c;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = pk2<false>(s[2 * i], s[2 * i + 1]);
    } else if constexpr (XK == 3) {
      const float* s = (const float*)x + r * x_stride + c;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = pk2<true>(s[2 * i], s[2 * i + 1]);
    } else {
      const uint16_t* s = (const uint16_t*)x + r * x_stride + c;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = (uint32_t)s[2 * i] | ((uint32_t)s[2 * i + 1] << 16);
    }
    *(uint4*)(xo + r * k + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int FMT, bool BF>
hipError_t launch_pf(const void* w, int num_experts, int64_t n, int64_t k, const uint16_t* x, int64_t x_stride,
                     const int32_t* chunks, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                     float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  using S = PfShape<FMT>;
  const int64_t rb = S::KQ ? k / 256 * S::BB : k / 32 * S::BB;
  const int64_t estride = n * rb;
  // chunk slots: with entries grouped by expert at most size_m/64 + experts
  // chunks; more (entries in any order) are taken by the workgroups in turn
  const int64_t runs_max = size_m < num_experts ? size_m : num_experts;
  int64_t gy = (size_m + kPfM - 1) / kPfM + runs_max;
  gy = gy < 1 ? 1 : gy > 65535 ? 65535 : gy;
  const dim3 grid((unsigned)((n + kPfNT - 1) / kPfNT), (unsigned)gy);
  constexpr auto* kfn = &moe_pf_kernel<FMT, BF>;
  if (S::Lds > 65536 && set_max_dynamic_lds<kfn>() != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * kPfW, S::Lds, st>>>((const uint8_t*)w, n, k, rb, estride, num_experts, x, x_stride, chunks, ids,
                                       topk_w, topk, (int)size_m, dst, ldd);
  return hipGetLastError();
}

template <bool BF>
hipError_t launch_pf_type(int type, const void* w, int num_experts, int64_t n, int64_t k, const uint16_t* x,
                          int64_t x_stride, const int32_t* chunks, const int32_t* ids, const float* topk_w, int topk,
                          int64_t size_m, float* dst, int64_t ldd, hipStream_t st) {
#define QMM_PF(F) launch_pf<F, BF>(w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk, size_m, dst, ldd, st)
  switch (type) {
    case T_Q4_K: return QMM_PF(T_Q4_K);
    case T_Q6_K: return QMM_PF(T_Q6_K);
    case T_Q8_0: return QMM_PF(T_Q8_0);
    case T_IQ4_NL: return QMM_PF(T_IQ4_NL);
    case T_MXFP4: return QMM_PF(T_MXFP4);
    default: return hipErrorInvalidValue;
  }
#undef QMM_PF
}

}  // namespace

bool moe_pf_supported(int type, int64_t k) {
  if (type == T_Q4_K || type == T_Q6_K) return k % 256 == 0 && k >= 256;
  return (type == T_Q8_0 || type == T_IQ4_NL || type == T_MXFP4) && k % 32 == 0 && k >= 32;
}

bool moe_pf_weights_ok(int type, const void* w) {
  // Q4_K stages copy whole 16-byte pieces of the rows
  return type != T_Q4_K || ((uintptr_t)w & 15) == 0;
}

int64_t moe_pf_row_bytes(int type, int64_t k) {
  switch (type) {
    case T_Q4_K: return k / 256 * 144;
    case T_Q6_K: return k / 256 * 210;
    case T_Q8_0: return k / 32 * 34;
    case T_IQ4_NL: return k / 32 * 18;
    case T_MXFP4: return k / 32 * 17;
    default: return -1;
  }
}

size_t moe_pf_chunks_bytes(int64_t size_m) {
  return (size_t)(1 + 3 * (size_m + size_m / kPfM + 1)) * sizeof(int32_t);
}

hipError_t launch_moe_pf_prep(const int32_t* expert_ids, int64_t size_m, int32_t* runs, int32_t* chunks,
                              const void* x, int x_kind, int64_t x_stride, int64_t k, int64_t rows, uint16_t* xo,
                              int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  // x_kind: -1 no conversion (the tables only), 0 f16 / 1 bf16 copied,
  // 2 f32 to f16, 3 f32 to bf16
  int64_t blocks = 0;
  if (x_kind >= 0) {
    const int64_t groups = rows * (k / 8);
    blocks = (groups + kPfPrepThreads - 1) / kPfPrepThreads;
    const int64_t cap = 8 * (int64_t)(cus > 0 ? cus : 256);
    blocks = blocks < cap ? blocks : cap;
  }
  const dim3 grid((unsigned)(1 + blocks));
  switch (x_kind) {
    case 2:
      moe_pf_prep_kernel<2><<<grid, kPfPrepThreads, 0, st>>>(expert_ids, (int)size_m, runs, chunks, x, x_stride, k,
                                                             rows, xo);
      break;
    case 3:
      moe_pf_prep_kernel<3><<<grid, kPfPrepThreads, 0, st>>>(expert_ids, (int)size_m, runs, chunks, x, x_stride, k,
                                                             rows, xo);
      break;
    default:
      moe_pf_prep_kernel<0><<<grid, kPfPrepThreads, 0, st>>>(expert_ids, (int)size_m, runs, chunks, x, x_stride, k,
                                                             rows, xo);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_moe_pf(int type, bool bf16, const void* w, int num_experts, int64_t n, int64_t k, const uint16_t* x,
                         int64_t x_stride, const int32_t* chunks, const int32_t* ids, const float* topk_w, int topk,
                         int64_t size_m, float* dst, int64_t ldd, hipStream_t st) {
  if (!moe_pf_weights_ok(type, w)) return hipErrorInvalidValue;
  return bf16 ? launch_pf_type<true>(type, w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk, size_m, dst,
                                     ldd, st)
              : launch_pf_type<false>(type, w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk, size_m, dst,
                                      ldd, st);
}

}  // namespace qmm
