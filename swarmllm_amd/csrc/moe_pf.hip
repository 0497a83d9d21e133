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
// up to 32 entries of one expert, in a table written by the one-workgroup
// prologue launch (moe_pf_prep_kernel). A workgroup takes a chunk and a tile
// of 32 x waves weight rows of the chunk's expert and walks k in stages of
// 256 values. For each stage, direct global-to-LDS copies bring each weight
// row's bytes of the stage (its 16-byte aligned window) and the chunk's 32
// input rows (256 values each, 16-byte pieces XOR-swizzled by row) into one
// half of double buffers while the waves work on the other half. Each wave
// owns 32 weight rows: lane L dequantizes row L%32 into the B operand of
// v_mfma_f32_32x32x16_{f16,bf16} (the chunk's entries are the A side), 16
// steps a stage. The order in which a stage's 256 values enter the steps is
// chosen per format so that a lane's 8 values of a step come from 8
// consecutive bytes of its row; the A side reads the input values of the same
// positions, and any order gives the same sum of products.
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

constexpr int kPfM = 32;                   // routing entries a chunk: the MFMA's M
constexpr int kPfK = 256;                  // values a stage
constexpr int kPfABytes = kPfM * kPfK * 2;  // the input tile of a stage (16-bit values)
constexpr int kPfACopies = kPfABytes / 1024;
constexpr int kPfPrepThreads = 256;

// Bytes of a weight row's stage (256 values), the 16-byte pieces of its window
// (aligned: the stage starts on a 16-byte boundary), the LDS row stride in
// pieces (odd, so that the 32 rows a wave reads in one instruction fall on
// distinct banks), waves, and the weight buffer of a stage.
template <int FMT, bool AL>
struct PfShape {
  static constexpr int SB = FMT == T_Q4_K ? 144 : FMT == T_Q6_K ? 210 : FMT == T_Q8_0 ? 272 : FMT == T_IQ4_NL ? 144 : 136;
  static constexpr int P = AL ? SB / 16 : (SB + 30) / 16;
  static constexpr int Ps = P | 1;
  static constexpr int W = FMT == T_Q8_0 ? 4 : 8;
  static constexpr int NT = 32 * W;
  static constexpr int WCopies = (NT * Ps + 63) / 64;
  static constexpr int WBytes = WCopies * 1024;
  static constexpr int Lds = 2 * kPfABytes + 2 * WBytes + 3 * kPfM * 4;
  static_assert(!AL || SB % 16 == 0, "aligned stages are whole pieces");
  static_assert(Lds <= 160 * 1024, "one workgroup's buffers fit a CU's LDS");
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

template <bool AL, int N>
__device__ __forceinline__ void lds_get(const uint8_t* win, int off, uint32_t* out) {
  if constexpr (AL && N == 4) {
    const uint4 v = *(const uint4*)(win + off);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else if constexpr (AL && N == 2) {
    const uint2 v = *(const uint2*)(win + off);
    out[0] = v.x;
    out[1] = v.y;
  } else {
    lds_words<N>(win, off, out);
  }
}

// One stage of a weight row for lane half h, from the row's window at byte o:
// step(piece, b) for each of its 16 steps, `piece` the 8-value group (of the
// stage's 32) whose values b holds. nb_left = the row's 32-value blocks from
// this stage on (32-value formats: blocks past the row are skipped).
template <int FMT, bool AL, bool BF, class Step>
__device__ __forceinline__ void pf_stage(const uint8_t* win, int o, int h, int nb_left, uint32_t t0, uint32_t t1,
                                         uint32_t t2, uint32_t t3, Step&& step) {
  if constexpr (FMT == T_Q4_K) {
    // d, dmin, 12 scale bytes, then qs[128]: value 64p + l is the low nibble
    // of qs[32p + l], value 64p + 32 + l its high nibble (l < 32); sub-block
    // j = 2p (low) and 2p + 1 (high) scale d * sc_j, offset dmin * m_j
    // (k_quants.rs to_float of BlockQ4K). Lane half h takes bytes
    // 32p + 16h .. +15: steps t = 0, 1 the low nibbles of its bytes 0-7, 8-15,
    // t = 2, 3 the high nibbles.
    uint32_t hd[4];
    lds_get<AL, 4>(win, o, hd);
    const float d = h2f((uint16_t)(hd[0] & 0xFFFF)), dm = h2f((uint16_t)(hd[0] >> 16));
    auto sb = [&](int i) { return (int)((hd[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF); };
#pragma unroll
    for (int p = 0; p < 4; p++) {
      int sc[2], mn[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int j = 2 * p + u;
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
      uint32_t q[4];
      lds_get<AL, 4>(win, o + 16 + 32 * p + 16 * h, q);
      step(8 * p + 2 * h, deq8<BF>(q[0] & 0x0F0F0F0Fu, q[1] & 0x0F0F0F0Fu, d1a, -m1a));
      step(8 * p + 2 * h + 1, deq8<BF>(q[2] & 0x0F0F0F0Fu, q[3] & 0x0F0F0F0Fu, d1a, -m1a));
      step(8 * p + 4 + 2 * h, deq8<BF>(q[0] & 0xF0F0F0F0u, q[1] & 0xF0F0F0F0u, d1b, -m1b));
      step(8 * p + 4 + 2 * h + 1, deq8<BF>(q[2] & 0xF0F0F0F0u, q[3] & 0xF0F0F0F0u, d1b, -m1b));
    }
  } else if constexpr (FMT == T_Q6_K) {
    // ql[128], qh[64], sc[16] (int8), d: in half g (values 128g ..), value
    // 128g + 32j + l (l < 32) is the 6-bit code of ql[64g + 32(j&1) + l]'s
    // low (j < 2) or high nibble and bits 2j, 2j+1 of qh[32g + l], minus 32,
    // times d * sc[8g + l/16 + 2j] (to_float of BlockQ6K). Lane half h takes
    // l = 16u + 8h .. +7.
    uint32_t scw[4];
    lds_words<4>(win, o + 192, scw);
    const float d = h2f((uint16_t)lds_u16(win, o + 208));
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int u = 0; u < 2; u++) {
        uint32_t A[2], B[2], H[2];
        lds_words<2>(win, o + 64 * g + 16 * u + 8 * h, A);
        lds_words<2>(win, o + 64 * g + 32 + 16 * u + 8 * h, B);
        lds_words<2>(win, o + 128 + 32 * g + 16 * u + 8 * h, H);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t* src = (j & 1) ? B : A;
          uint32_t c[2];
#pragma unroll
          for (int w = 0; w < 2; w++) {
            const uint32_t nib = (j & 2) ? ((src[w] >> 4) & 0x0F0F0F0Fu) : (src[w] & 0x0F0F0F0Fu);
            c[w] = nib | (((H[w] >> (2 * j)) & 0x03030303u) << 4);
          }
          const int si = 8 * g + u + 2 * j;
          const float ds = d * (float)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFF);
          // ds (code - 32) as one rounding of ds * code - 32 ds
          step(16 * g + 4 * j + 2 * u + h, deq8<BF>(c[0], c[1], ds, -32.0f * ds));
        }
      }
  } else {
    // 8 blocks of 32 values. Q8_0: f16 d, 32 int8 codes; lane half h takes
    // codes 16t + 8h .. +7 for steps t = 0, 1. IQ4_NL (f16 d) and MXFP4 (e8m0
    // scale, halved against the doubled table): value l < 16 the low nibble of
    // qs[l], 16 + l the high; lane half h takes qs[8h .. 8h+7], the low
    // nibbles at t = 0, the high at t = 1. Signed codes are read as
    // unsigned (code + 128) and fma(d, code + 128, -128 d): exact.
    constexpr int B = FMT == T_Q8_0 ? 34 : FMT == T_IQ4_NL ? 18 : 17;
    constexpr int Head = FMT == T_MXFP4 ? 1 : 2;
#pragma unroll
    for (int b = 0; b < 8; b++) {
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
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const uint32_t c0 = (uint32_t)lut16(t ? (q[0] >> 4) & 0x0F0F0F0Fu : q[0] & 0x0F0F0F0Fu, t0, t1, t2, t3);
          const uint32_t c1 = (uint32_t)lut16(t ? (q[1] >> 4) & 0x0F0F0F0Fu : q[1] & 0x0F0F0F0Fu, t0, t1, t2, t3);
          step(4 * b + 2 * t + h, deq8<BF>(c0 ^ 0x80808080u, c1 ^ 0x80808080u, d, -128.0f * d));
        }
      }
    }
  }
}

template <int FMT, bool AL, bool BF>
__global__ __launch_bounds__((64 * PfShape<FMT, AL>::W)) void moe_pf_kernel(
    const uint8_t* __restrict__ W, int64_t n, int64_t k, int64_t rb, int64_t estride, int num_experts,
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ chunks,
    const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int topk, int size_m, float* __restrict__ dst,
    int64_t ldd) {
  using S = PfShape<FMT, AL>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const sA = smem;                          // [2][32 rows][512 B]
  uint8_t* const sW = smem + 2 * kPfABytes;          // [2][WBytes]
  int* const s_in = (int*)(sW + 2 * S::WBytes);      // the chunk's input rows
  int* const s_out = s_in + kPfM;                    // output rows (-1: none)
  float* const s_sc = (float*)(s_out + kPfM);        // routing weights

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * S::NT;
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

    // The copies of stage st into buffer half `buf`: weight copy i moves
    // window pieces f = 64 i + L (row f / Ps, piece f % Ps of the aligned
    // window at or before the row's stage, clamped to the piece holding the
    // stage's last byte in the row); input copy i moves rows 2i, 2i + 1, lane
    // L writing position L % 32 of row m = 2i + L/32, which holds piece
    // (L % 32) ^ m of the row's stage (clamped to the row's last piece). The
    // waves take copies wv, wv + W, ...
    auto issue = [&](int st, int buf) {
      for (int j = wv; j < S::WCopies + kPfACopies; j += S::W) {
        if (j < S::WCopies) {
          const uint32_t f = 64u * (uint32_t)j + (uint32_t)lane;
          const uint32_t r = f / (uint32_t)S::Ps < (uint32_t)S::NT ? f / (uint32_t)S::Ps : S::NT - 1;
          const int64_t gr = n0 + r < n ? n0 + r : n - 1;
          const uint32_t rs = (uint32_t)(gr * rb);
          const uint32_t a = rs + (uint32_t)(S::SB * st);
          const uint32_t send = a + S::SB < rs + (uint32_t)rb ? a + S::SB : rs + (uint32_t)rb;
          const uint32_t first = a & ~15u, last = (send - 1u) & ~15u;
          const uint32_t off = first + 16u * (f % (uint32_t)S::Ps);
          dma16(We, off < last ? off : last,
                __builtin_amdgcn_readfirstlane(lds_addr(sW + buf * S::WBytes + 1024 * j)));
        } else {
          const int i = j - S::WCopies;
          const int m = 2 * i + (lane >> 5);
          const uint32_t q = (uint32_t)((lane & 31) ^ m);
          const uint32_t el = (uint32_t)(kPfK * st) + 8u * q;
          const uint32_t cl = el < (uint32_t)k - 8u ? el : (uint32_t)k - 8u;
          dma16(x, 2u * ((uint32_t)s_in[m] * (uint32_t)x_stride + cl),
                __builtin_amdgcn_readfirstlane(lds_addr(sA + buf * kPfABytes + 1024 * i)));
        }
      }
    };

    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    pf_f16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    for (int st = 0; st < nst; st++) {
      const int cur = st & 1;
      if (st + 1 < nst) issue(st + 1, cur ^ 1);
      const uint8_t* win = sW + cur * S::WBytes + (32 * wv + r32) * (S::Ps * 16);
      const int o = AL ? 0 : (int)((wrow_off + (uint32_t)(S::SB * st)) & 15u);
      const uint8_t* arow = sA + cur * kPfABytes + r32 * 512;
      pf_stage<FMT, AL, BF>(win, o, h, nb32 - 8 * st, t0, t1, t2, t3, [&](int piece, pf_u4 b) {
        const pf_u4 a = *(const pf_u4*)(arow + 16 * (piece ^ r32));
        acc = mfma16<BF>(a, b, acc);
      });
      // the next stage has landed, and every wave is done with this one
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    // lane L holds entries m = 8 (i/4) + 4 h + i%4 of weight row r32
    const int64_t col = n0 + 32 * wv + r32;
    if (col < n) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int m = 8 * (i >> 2) + 4 * h + (i & 3);
        const int p = s_out[m];
        if (p >= 0) dst[(int64_t)p * ldd + col] = __fmul_rn(acc[i], s_sc[m]);
      }
    }
    __syncthreads();  // the entry tables are rewritten by the next chunk
  }
}

// Block 0: the run table and the chunk table of 32 entries. Blocks 1..: the
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

template <int FMT, bool AL, bool BF>
hipError_t launch_pf(const void* w, int num_experts, int64_t n, int64_t k, const uint16_t* x, int64_t x_stride,
                     const int32_t* chunks, const int32_t* ids, const float* topk_w, int topk, int64_t size_m,
                     float* dst, int64_t ldd, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  using S = PfShape<FMT, AL>;
  const int64_t rb = FMT == T_Q4_K ? k / 256 * 144 : FMT == T_Q6_K ? k / 256 * 210 : k / 32 * (S::SB / 8);
  const int64_t estride = n * rb;
  // chunk slots: with entries grouped by expert at most size_m/32 + experts
  // chunks; more (entries in any order) are taken by the workgroups in turn
  const int64_t runs_max = size_m < num_experts ? size_m : num_experts;
  int64_t gy = (size_m + kPfM - 1) / kPfM + runs_max;
  gy = gy < 1 ? 1 : gy > 65535 ? 65535 : gy;
  const dim3 grid((unsigned)((n + S::NT - 1) / S::NT), (unsigned)gy);
  auto* kfn = &moe_pf_kernel<FMT, AL, BF>;
  if (set_max_dynamic_lds((const void*)kfn) != hipSuccess) return hipErrorInvalidValue;
  kfn<<<grid, 64 * S::W, S::Lds, st>>>((const uint8_t*)w, n, k, rb, estride, num_experts, x, x_stride, chunks, ids,
                                       topk_w, topk, (int)size_m, dst, ldd);
  return hipGetLastError();
}

template <bool BF>
hipError_t launch_pf_type(int type, bool aligned, const void* w, int num_experts, int64_t n, int64_t k,
                          const uint16_t* x, int64_t x_stride, const int32_t* chunks, const int32_t* ids,
                          const float* topk_w, int topk, int64_t size_m, float* dst, int64_t ldd, hipStream_t st) {
#define QMM_PF(F, A) \
  launch_pf<F, A, BF>(w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk, size_m, dst, ldd, st)
  switch (type) {
    case T_Q4_K: return aligned ? QMM_PF(T_Q4_K, true) : QMM_PF(T_Q4_K, false);
    case T_Q6_K: return QMM_PF(T_Q6_K, false);
    case T_Q8_0: return QMM_PF(T_Q8_0, false);
    case T_IQ4_NL: return aligned ? QMM_PF(T_IQ4_NL, true) : QMM_PF(T_IQ4_NL, false);
    case T_MXFP4: return QMM_PF(T_MXFP4, false);
    default: return hipErrorInvalidValue;
  }
#undef QMM_PF
}

}  // namespace

bool moe_pf_supported(int type, int64_t k) {
  if (type == T_Q4_K || type == T_Q6_K) return k % 256 == 0 && k >= 256;
  return (type == T_Q8_0 || type == T_IQ4_NL || type == T_MXFP4) && k % 32 == 0 && k >= 32;
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
  // whole-piece stages: 16-byte aligned weights whose rows hold whole stages
  // of a multiple of 16 bytes
  const bool aligned = ((uintptr_t)w & 15) == 0 && k % 256 == 0;
  return bf16 ? launch_pf_type<true>(type, aligned, w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk,
                                     size_m, dst, ldd, st)
              : launch_pf_type<false>(type, aligned, w, num_experts, n, k, x, x_stride, chunks, ids, topk_w, topk,
                                      size_m, dst, ldd, st);
}

}  // namespace qmm
