// gemm_q4k_sp.hip — Q4_K prefill GEMM in ONE int8 matrix-core pass (gfx950).
//
// dst[m][n] = sum over super-blocks of  d_n dy_m sum_j sc_nj sum_{i in j} q_ni y_mi
//                                      - dmin_n dy_m sum_j m_nj S_mj
// is candle's Q4_K x Q8_K vec_dot (vendor/candle/candle-core/src/quantized/
// k_quants.rs:2031-2111) against the activation quantized as the reference
// quantizes it for Q4_K (BlockQ8K::from_float, :2882-2927): per-256 scale
// dy_m, int8 codes y, S_mj the code sum of 32-value sub-block j.
//
// One pass instead of two. sc*q needs 10 bits and an int8 operand holds 8,
// so the weight enters the matrix cores as
//     w8 = floor((sc (q - 8) + 2) / 4)   in [-126, 110],
// sc (q - 8) rounded to a multiple of 4. Then
//     sum_j sc_j sum q y  ~=  4 sum w8 y  +  8 sum_j sc_j S_j ,
// where the second sum (the -8 offset) is exact and joins the min term in
// one f16 product per super-block:
//     sum_j S_j * (8 d sc_j - dmin m_j)   (A = dy S_j, B = 8 d sc_j - dmin m_j).
// The rounding of sc (q - 8) (|error| <= 2 of a code step of 4) is the
// kernel's one approximation beyond the f16 operands of that product; the
// normalised error |y - y_ref| / (||w|| ||x||) stays near 4e-4 at most on C3
// with its outlier channels, inside the 2e-3 bound of the GEMM.
//
// Integer accumulators start at the bits of 1.5 * 2^23, so after a
// super-block's eight MFMAs each holds the f32 1.5 * 2^23 + T exactly
// (|T| < 2^22); the epilogue folds it with one fma, acc += (1.5 2^23 + T) s,
// and the same f16 product that carries the min term subtracts
// 1.5 * 2^23 * s (its spare K slots, s = 4 d dy as two f16 halves x d).
//
// Each row's activation scales are divided by a power of two 2^e_m (the
// largest |dy| of the row in [0.5, 1)), which keeps the f16 operands of the
// per-super-block product in range for activations of any size; the output
// is multiplied back by 2^e_m (exact).
//
// Data movement (workgroup: 8 waves, 256 rows x 128 weight rows, each wave
// 64 x 64 as 2 x 2 tiles of v_mfma_i32_32x32x32_i8):
//   - K is staged 128 values (half a super-block) at a time. The activation
//     codes of the stage (256 rows x 128 B) and the raw Q4_K bytes of the
//     super-block (128 rows x 144 B) reach LDS by direct global-to-LDS copies,
//     one stage ahead into the other half of double buffers.
//   - The workgroup's 512 threads turn the next stage's raw nibbles into int8
//     w8 in LDS (each thread 32 values: four packed 16-bit multiply-adds per
//     8 values, then a byte permute), beside the current stage's MFMAs. The
//     weights are expanded once per 256 activation rows.
//   - The f16 product operands, dy and d of a super-block are written to LDS
//     by the threads during its first half and read by its epilogue.
// Rows past M and weight rows past N are read as the last row (valid
// memory); their outputs are never stored.
#include "lds_copy.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128;  // workgroup tile: activation rows x weight rows
constexpr int kThreads = 512;        // 8 waves: 4 (rows) x 2 (weight rows), 64 x 64 each
constexpr int kStage = 128;          // K values a stage (half a super-block)
constexpr uint32_t kMagic = 0x4B400000u;  // bits of 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;
// exponent shift of the f16 operands: A carries 2^-8, B 2^8
constexpr float kToA = 1.0f / 256.0f, kToB = 256.0f;

__device__ __forceinline__ uint32_t pkmad(uint32_t a, uint32_t b, uint32_t c) {
  const u16x2 x = __builtin_bit_cast(u16x2, a), y = __builtin_bit_cast(u16x2, b), z = __builtin_bit_cast(u16x2, c);
  return __builtin_bit_cast(uint32_t, x * y + z);
}

__device__ __forceinline__ uint32_t word(const uint4& c, int e) {
  return e == 0 ? c.x : e == 1 ? c.y : e == 2 ? c.z : c.w;
}

// A staged tile keeps 128 bytes a row; its 16-byte piece p of row r sits at
// piece p ^ swz(r), so the 16 rows one 16-lane group of an MFMA operand read
// (rows r0 .. r0+15, one piece each) cover the 64 LDS banks once.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r >> 1) & 7u; }

// LDS access by byte address. The kernel keeps per-lane byte offsets that it
// makes opaque once a stage (`opaque`), so the compiler forms each address
// as offset + the buffer's constant address (an instruction immediate)
// instead of keeping one precomputed address per buffer and K-step live.
typedef int lds_i4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ T lds_ld(uint32_t a) { return *(const __attribute__((address_space(3))) T*)(uintptr_t)a; }
template <typename T>
__device__ __forceinline__ void lds_st(uint32_t a, const T& v) { *(__attribute__((address_space(3))) T*)(uintptr_t)a = v; }
__device__ __forceinline__ uint4 lds_ld4(uint32_t a) {
  const lds_i4 v = lds_ld<lds_i4>(a);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ void lds_st4(uint32_t a, const uint4& v) {
  lds_st<lds_i4>(a, lds_i4{(int)v.x, (int)v.y, (int)v.z, (int)v.w});
}
__device__ __forceinline__ void opaque(uint32_t& v) { asm volatile("" : "+v"(v)); }

// 2^-e with |v| in [2^(e-1), 2^e) for the largest |v| of a row: the factor
// that brings the row's scales into [0.5, 1); 1 for a zero or non-finite row.
__device__ __forceinline__ float row_factor(float maxabs) {
  const uint32_t E = (__builtin_bit_cast(uint32_t, maxabs) >> 23) & 0xFFu;
  if (maxabs == 0.0f || E == 0xFFu) return 1.0f;
  const int fe = 253 - (int)E;  // biased exponent of 2^(126 - E)
  return __builtin_bit_cast(float, (uint32_t)(fe < 1 ? 1 : (fe > 254 ? 254 : fe)) << 23);
}
// 1 / r for a row factor r = 2^p (biased exponent 1..252): 2^-p, a normal
// float, so x * inv_pow2(r) is x / r exactly (both scale x by 2^-p and round
// once), without a division.
__device__ __forceinline__ float inv_pow2(float r) {
  return __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, r));
}

// The launch's weights (up to kMaxTargets sharing one activation) and their
// K splits; see launch_gemm_q4k_sp_targets.
struct SpArgs {
  const void* w[kMaxTargets];
  float* dst[kMaxTargets];
  int64_t ldd[kMaxTargets];
  int64_t n[kMaxTargets];
  int unit_end[kMaxTargets];   // workgroups of weights 0..t
  int splits[kMaxTargets];     // K splits of weight t's tiles (1, 2 or 4)
  int per[kMaxTargets];        // consecutive splits a workgroup computes (1, or 2 / 4 for Q4_K)
  int tile_base[kMaxTargets];  // the sum kernel's first workgroup for weight t (its split tiles before it)
  int64_t part_off[kMaxTargets];  // its first slot in `part` (floats)
  const int8_t* yq;
  const float* yd;
  const int16_t* ybs;
  int64_t M;
  float* part;    // split slots: tiles x splits x 256 x 128 f32
  int nsb, mtiles, remap;
};

// The raw bytes of one weight row's super-block in LDS: Q4_K's 144-byte
// blocks (9 aligned pieces), Q6_K's 210-byte blocks as the 14 aligned
// 16-byte pieces around them (rows 16-byte aligned: k a multiple of 2048).
template <int FMT>
struct SpFmt {
  static constexpr bool kQ6 = FMT == T_Q6_K;
  static constexpr int kBlock = kQ6 ? 210 : 144;  // bytes of a super-block
  static constexpr int kRaw = kQ6 ? 224 : 144;    // LDS bytes of a row's super-block
  static constexpr int kPieces = kRaw / 16;       // 16-byte copies a row
  static constexpr int kCopies = kBN * kPieces / 64;  // 64-lane copies a super-block: 18 / 28
  static constexpr int kWaveCopies = (kCopies + 7) / 8;  // a wave's share: 3 / 4
};
// Q6_K's weight enters as w8 = round(m_j (q - 32) / 256) with the integer
// multiplier m_j = round(127 sc_j / 16): |m_j (q - 32)| <= 1016 * 32 fits the
// 16-bit lanes for every int8 sc_j (-128 included), and the super-block's
// scale becomes d * 256 * 16 / 127.
constexpr float kQ6Eff = 4096.0f / 127.0f;

// One thread's 32 values of a Q6_K stage (half `half` of super-block sbx,
// the layout of BlockQ6K::to_float,
// vendor/candle/candle-core/src/quantized/k_quants.rs:2657-2727): the 16
// values of sub-block part p of 32-value group c (low nibbles of ql chunk c,
// qh bits 2c) and of group c + 2 (high nibbles of the same ql bytes, qh bits
// 2c + 4), into int8 pieces 2c + p and 2c + p + 4 of the row at w0 and w1.
// The four dwords of each piece are formed in the order rho, rho + 1, ...
// (rho = (row / 4) mod 4): the 16 rows a wave expands lie 224 bytes apart
// in LDS, and reading the same dword of each would put them on 8 banks;
// rotated, they spread over all of them.
// wr: the row's window in LDS (the block at byte (2 sbx) mod 16 of it).
// t: the thread's index (c = bit 1, p = bit 0, its row t / 4).
__device__ __forceinline__ void build_q6(uint32_t wr, int half, uint32_t w0, uint32_t w1, int sbx, uint32_t t) {
  const uint32_t c = (t >> 1) & 1u, p = t & 1u, rho = (t >> 4) & 3u;
  const uint32_t boff = (2u * (uint32_t)sbx) & 15u;
  const uint32_t al = boff & 3u;  // 0 or 2: the blocks sit 2-byte aligned in their windows
  const uint32_t wb = wr + (boff & 12u);  // the dword holding the block's first byte
  const uint32_t ql4 = wb + 64u * (uint32_t)half + 32u * c + 16u * p;
  const uint32_t qh4 = wb + 128u + 32u * (uint32_t)half + 16u * p;
  // sub-block scales 8 half + 2c + p and 8 half + 2c + p + 4: bytes o and
  // o + 4 past the scales' first dword (o <= 5), the same byte of two dwords
  const uint32_t o = al + 2u * c + p;
  const uint32_t sa = wb + 192u + 8u * (uint32_t)half + (o & ~3u);
  const uint32_t sh = 8u * (o & 3u);
  const int sc0 = (int)(int8_t)((lds_ld<uint32_t>(sa) >> sh) & 0xFFu);
  const int sc1 = (int)(int8_t)((lds_ld<uint32_t>(sa + 4u) >> sh) & 0xFFu);
  const int m0 = (127 * sc0 + 8) >> 4, m1 = (127 * sc1 + 8) >> 4;  // round(127 sc / 16)
  // per 16-bit lane: m (q - 32) + 128, whose high byte is w8
  const uint32_t M0 = ((uint32_t)m0 & 0xFFFFu) * 0x10001u, C0 = ((uint32_t)(128 - 32 * m0) & 0xFFFFu) * 0x10001u;
  const uint32_t M1 = ((uint32_t)m1 & 0xFFFFu) * 0x10001u, C1 = ((uint32_t)(128 - 32 * m1) & 0xFFFFu) * 0x10001u;
  const uint32_t lsh = 4u - 2u * c, hsh = 2u * c;  // qh bits 2c and 2c + 4 to bits 4-5
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t d4 = 4u * (((uint32_t)i + rho) & 3u);
    const uint32_t lw = __builtin_amdgcn_alignbyte(lds_ld<uint32_t>(ql4 + d4 + 4u), lds_ld<uint32_t>(ql4 + d4), al);
    const uint32_t hw = __builtin_amdgcn_alignbyte(lds_ld<uint32_t>(qh4 + d4 + 4u), lds_ld<uint32_t>(qh4 + d4), al);
    const uint32_t qa = (lw & 0x0F0F0F0Fu) | ((hw << lsh) & 0x30303030u);
    const uint32_t qb = ((lw >> 4) & 0x0F0F0F0Fu) | ((hw >> hsh) & 0x30303030u);
    const uint32_t ea = pkmad(qa & 0x00FF00FFu, M0, C0), oa = pkmad((qa >> 8) & 0x00FF00FFu, M0, C0);
    const uint32_t eb = pkmad(qb & 0x00FF00FFu, M1, C1), ob = pkmad((qb >> 8) & 0x00FF00FFu, M1, C1);
    lds_st<uint32_t>(w0 + d4, __builtin_amdgcn_perm(oa, ea, 0x07030501u));
    lds_st<uint32_t>(w1 + d4, __builtin_amdgcn_perm(ob, eb, 0x07030501u));
  }
}

template <int FMT>
__global__ __launch_bounds__(kThreads, 1) void gemm_kq_sp_kernel(const SpArgs a) {
  using F = SpFmt<FMT>;
  constexpr bool Q6 = F::kQ6;
  // Each half of each double buffer is its own object and the stage loop is
  // unrolled over two super-blocks, so every access names its buffer
  // statically (the compiler can tell reads of one half from writes of the other).
  __shared__ __attribute__((aligned(16))) int8_t s_a0[kBM * kStage], s_a1[kBM * kStage];
  __shared__ __attribute__((aligned(16))) int8_t s_b0[kBN * kStage], s_b1[kBN * kStage];
  __shared__ __attribute__((aligned(16))) uint8_t s_w0[kBN * F::kRaw], s_w1[kBN * F::kRaw];
  // Q4_K: the f16 product's operands of a super-block (Q6_K forms its
  // operands from s_dy and s_d4 in registers)
  __shared__ __attribute__((aligned(16))) _Float16 s_rop[Q6 ? 1 : kBM][16];
  __shared__ __attribute__((aligned(16))) _Float16 s_cop[Q6 ? 1 : kBN][16];
  __shared__ __attribute__((aligned(16))) float s_dy[kBM];          // Q4_K dy_m 2^-e_m; Q6_K its f16 value
  __shared__ __attribute__((aligned(16))) float s_d4[kBN];          // Q4_K 4 d_n; Q6_K dq_n (f16 value)
  __shared__ __attribute__((aligned(16))) float s_rf[kBM];          // 2^-e_m
  // a super-block's activation sums (bsums) and scales, copied one stage
  // ahead of the stage that turns them into the f16 operands
  __shared__ __attribute__((aligned(16))) int16_t s_bsr[Q6 ? 8 : kBM * 16];
  __shared__ __attribute__((aligned(16))) float s_ydr[kBM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv & 3, wn = wv >> 2;
  const int h = lane >> 5, r32 = lane & 31;

  // workgroup -> (weight, tile, K split); the row tiles and splits of one
  // weight tile on one XCD (its L2). Units are numbered weight after weight:
  // weight t holds units [unit_end[t-1], unit_end[t]), each of its tiles
  // `splits[t]` consecutive K ranges times the row tiles.
  const int total = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  const int idx = a.remap ? (b & 7) * (total >> 3) + (b >> 3) : b;
  const int t = idx < a.unit_end[0] ? 0 : idx < a.unit_end[1] ? 1 : idx < a.unit_end[2] ? 2 : 3;
  // fields of weight t by selects (a dynamic index into the argument arrays
  // would copy them to private memory)
  auto pick = [&](const auto& arr) { return t == 0 ? arr[0] : t == 1 ? arr[1] : t == 2 ? arr[2] : arr[3]; };
  const int u0 = t == 0 ? 0 : t == 1 ? a.unit_end[0] : t == 2 ? a.unit_end[1] : a.unit_end[2];
  const int S = pick(a.splits);
  const int P = Q6 ? 1 : pick(a.per);
  const int mtiles = a.mtiles;
  const int loc = idx - u0;
  // a weight's units: row tiles fastest, then column tiles, then the split
  // groups, so the units an XCD takes (consecutive, through the remap) share
  // one K range: the activation columns an XCD reads are M x K/S (C3's down
  // product, 512 x 14336 cut in 4: 1.8 MB an XCD, which its L2 holds; with
  // the splits fastest every XCD read the whole 7.3 MB activation)
  const int64_t N = pick(a.n);
  const int ctiles = (int)((N + kBN - 1) / kBN);
  const int mt = loc % mtiles, rest = loc / mtiles;
  const int ct = rest % ctiles, split = (rest / ctiles) * P;
  const uint8_t* __restrict__ W = (const uint8_t*)pick(a.w);
  const int nsb = a.nsb;
  const int8_t* __restrict__ yq = a.yq;
  const float* __restrict__ yd = a.yd;
  const int16_t* __restrict__ ybs = a.ybs;
  const int64_t M = a.M;
  const int64_t m0 = (int64_t)mt * kBM;
  const int64_t n0 = (int64_t)ct * kBN;
  // this workgroup's super-blocks: splits split .. split + P - 1, each
  // plen super-blocks (nsb is a multiple of 2 S when S > 1)
  const int plen = nsb / S;
  const int sb0 = split * nsb / S, sb1 = (split + P) * nsb / S;

  const int64_t K = (int64_t)nsb * 256;
  const uint32_t rowbytes = (uint32_t)nsb * F::kBlock;

  // ---- per-lane byte offsets of the copies (stage 0 / super-block 0) ----
  // activation: 32 copies a stage, 8 rows each; wave wv takes copies wv + 8u
  // Copy u of this wave moves rows 64u + 8wv .. +7; lane L row 64u + 8wv +
  // L/8 (the swizzle of a row is the same 64 rows on), clamped to M - 1.
  const uint32_t arow_l = 8u * (uint32_t)wv + ((uint32_t)lane >> 3);
  const uint32_t a_rowk = (uint32_t)((m0 + arow_l) * K);  // < 2^31: rows + 256 rows of k
  const uint32_t a_lastk = (uint32_t)((M - 1) * K);
  const uint32_t a_piece = 16u * (((uint32_t)lane & 7u) ^ swz(arow_l));
  auto aoff = [&](int u) -> uint32_t {
    const uint32_t rk = a_rowk + (uint32_t)(64 * u) * (uint32_t)K;
    return (rk < a_lastk ? rk : a_lastk) + a_piece;
  };
  // weights: F::kCopies copies a super-block (128 rows x F::kPieces pieces),
  // copy i = wv + 8u; Q6_K's copies past the last repeat it (same LDS bytes)
  auto woff_of = [&](int u, uint32_t ln) -> uint32_t {
    const uint32_t i = (uint32_t)(wv + 8 * u);
    const uint32_t f = 64u * (i < (uint32_t)F::kCopies ? i : (uint32_t)F::kCopies - 1u) + ln;
    const uint32_t col = f / (uint32_t)F::kPieces;
    const int64_t gc = n0 + col < N ? n0 + col : N - 1;
    return (uint32_t)gc * rowbytes + 16u * (f - (uint32_t)F::kPieces * col);
  };
  // Q4_K keeps its three offsets; Q6_K forms its four at each use (from a
  // lane value the compiler cannot hoist), which keeps them out of registers
  uint32_t woff[F::kWaveCopies];
#pragma unroll
  for (int u = 0; u < F::kWaveCopies; u++) woff[u] = Q6 ? 0u : woff_of(u, (uint32_t)lane);
  // the per-super-block row inputs: bsums (32 bytes a row, 8 copies, one a
  // wave) and dy (4 bytes a row, 4 dword copies, waves 0-3)
  const uint32_t bsr = 32u * (uint32_t)wv + ((uint32_t)lane >> 1);
  const int64_t bsrow = m0 + bsr < M ? m0 + bsr : M - 1;
  const uint32_t bsoff = (uint32_t)(bsrow * (K / 16) * 2) + 16u * ((uint32_t)lane & 1u);
  const uint32_t ydr = 64u * (uint32_t)(wv & 3) + (uint32_t)lane;
  const int64_t ydrow = m0 + ydr < M ? m0 + ydr : M - 1;
  const uint32_t ydoff = (uint32_t)(ydrow * nsb) * 4u;
  auto dma_a1 = [&](int g, int8_t* sa, int u) {
    dma16(yq + 128 * (int64_t)g, aoff(u), lds_addr(sa + 1024 * (wv + 8 * u)));
  };
  auto dma_w1 = [&](int sb, uint8_t* sw, int u) {
    if constexpr (Q6) {
      const int i = wv + 8 * u < F::kCopies ? wv + 8 * u : F::kCopies - 1;
      uint32_t ln = (uint32_t)lane;
      asm volatile("" : "+v"(ln));
      dma16(W + 16 * ((210 * (int64_t)sb) >> 4), woff_of(u, ln), lds_addr(sw + 1024 * i));
    } else if (wv + 8 * u < F::kCopies) {
      dma16(W + 144 * (int64_t)sb, woff[u], lds_addr(sw + 1024 * (wv + 8 * u)));
    }
  };
  auto dma_rows = [&](int sb, int part) {
    if (Q6 && part == 0) return;  // Q6_K has no min term: no code sums
    if (part == 0)
      dma16((const uint8_t*)ybs + 32 * (int64_t)sb, bsoff, lds_addr((uint8_t*)s_bsr + 1024 * wv));
    else if (wv < 4)
      dma4(yd + sb, ydoff, lds_addr(s_ydr + 64 * wv));
  };

  // ---- expansion of a stage's weights: thread -> (weight row, piece) ----
  // Q4_K: 16 consecutive lanes: 16 rows, one piece. Q6_K: 4 consecutive
  // lanes a row (groups c, c + 2 of sub-block part p), 16 rows a wave.
  const int bn = Q6 ? tid >> 2 : tid & (kBN - 1), bpi = tid >> 7;
  // lane offsets of the expansion (made opaque once a stage): the raw row,
  // and the two 16-byte pieces it writes in the expanded row
  const uint32_t plo = Q6 ? (uint32_t)tid & 3u : 4u * ((uint32_t)bpi >> 1) + ((uint32_t)bpi & 1u);
  uint32_t x_raw = (uint32_t)bn * F::kRaw;
  uint32_t x_w0 = (uint32_t)bn * kStage + 16u * (plo ^ swz(bn));
  // (Q6_K: piece plo + 4, x_w0 ^ 64 since plo < 4; formed at each use)
  uint32_t x_w1 = Q6 ? 0u : (uint32_t)bn * kStage + 16u * ((plo + 2u) ^ swz(bn));
  auto build = [&](const uint8_t* sw, int half, int8_t* sbt, int sbx) {
    const uint32_t wr = lds_addr(sw) + x_raw, bt = lds_addr(sbt);
    if constexpr (Q6) {
      build_q6(wr, half, bt + x_w0, bt + (x_w0 ^ 64u), sbx, (uint32_t)tid);
      return;
    }
    // both reads in flight together: the second address is formed (opaque)
    // before the first read, else the compiler put it in the register of the
    // first read's unused dword 0 and waited for that read before issuing it
    uint32_t ra = wr + 16u * (uint32_t)(1 + 4 * half + bpi);
    opaque(ra);
    const uint4 hdr = lds_ld4(wr);
    const uint4 raw = lds_ld4(ra);
    // 6-bit scales of sub-blocks 4 half + 2 (bpi >> 1) and the next
    // (get_scale_min_k4, vendor/candle/candle-core/src/quantized/utils.rs:50-60)
    const uint32_t scw = half == 0 ? (hdr.y & 0x3f3f3f3fu)
                                   : ((hdr.w & 0x0f0f0f0fu) | (((hdr.y >> 6) & 0x03030303u) << 4));
    const uint32_t sw2 = scw >> (16 * (bpi >> 1));
    const uint32_t sc0 = sw2 & 0xFFu, sc1 = (sw2 >> 8) & 0xFFu;
    // per 16-bit lane: 64 sc (q - 8) + 128, whose high byte is w8
    const uint32_t mlo = (64u * sc0) * 0x10001u, blo = ((128u - 512u * sc0) & 0xFFFFu) * 0x10001u;
    const uint32_t mhi = (4u * sc1) * 0x10001u, bhi = ((128u - 512u * sc1) & 0xFFFFu) * 0x10001u;
    uint4 olo, ohi;
    uint32_t* lo = (uint32_t*)&olo;
    uint32_t* hi = (uint32_t*)&ohi;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t D = word(raw, e), D8 = D >> 8;
      const uint32_t el = pkmad(D & 0x000F000Fu, mlo, blo), ol = pkmad(D8 & 0x000F000Fu, mlo, blo);
      const uint32_t eh = pkmad(D & 0x00F000F0u, mhi, bhi), oh = pkmad(D8 & 0x00F000F0u, mhi, bhi);
      lo[e] = __builtin_amdgcn_perm(ol, el, 0x07030501u);
      hi[e] = __builtin_amdgcn_perm(oh, eh, 0x07030501u);
    }
    lds_st4(bt + x_w0, olo);
    lds_st4(bt + x_w1, ohi);
  };

  // ---- per-super-block scales: rows (threads 0-255), weight rows (256-383) ----
  const int64_t prow = m0 + (tid & 255) < M ? m0 + (tid & 255) : M - 1;
  auto prep = [&](const uint8_t* sw, int sbp) {
    if constexpr (Q6) {
      // rows: dy in f16 (row factor 2^-e / 2: at most 0.5, so dy 2^16 fits
      // f16); weight rows: dq = f16(d * 256 * 16 / 127 * 2^7)
      uint32_t t4 = 4u * (uint32_t)tid;  // opaque: the addresses are formed here, not kept live
      opaque(t4);
      if (tid < 256) {
        const float y = lds_ld<float>(lds_addr(s_ydr) + t4) * lds_ld<float>(lds_addr(s_rf) + t4);
        lds_st<float>(lds_addr(s_dy) + t4, (float)(_Float16)(y * 0.5f));
      } else if (tid < 256 + kBN) {
        const uint32_t n4 = t4 - 1024u;
        const uint16_t dh = lds_ld<uint16_t>(lds_addr(sw) + (n4 >> 2) * F::kRaw + ((2u * (uint32_t)sbp) & 15u) + 208u);
        lds_st<float>(lds_addr(s_d4) + n4, (float)(_Float16)(h2f(dh) * (kQ6Eff * 128.0f)));
      }
      return;
    }
    if (tid < 256) {
      const float dy = s_ydr[tid] * s_rf[tid];
      const uint4 pbs0 = *(const uint4*)&s_bsr[16 * tid], pbs1 = *(const uint4*)&s_bsr[16 * tid + 8];
      h8 a, c = {};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t wd = word(j < 4 ? pbs0 : pbs1, j & 3);
        const int s = (int)(int16_t)(wd & 0xFFFFu) + (int)(int16_t)(wd >> 16);
        a[j] = (_Float16)(dy * (float)s * kToA);
      }
      const float v = -kMagicF * dy * kToA;
      const _Float16 vh = (_Float16)v;
      c[0] = vh;
      c[1] = (_Float16)(v - (float)vh);
      *(h8*)&s_rop[tid][0] = a;
      *(h8*)&s_rop[tid][8] = c;
      s_dy[tid] = dy;
    } else if (tid < 256 + kBN) {
      const int n = tid - 256;
      const uint4 hdr = *(const uint4*)(sw + n * 144);
      const uint32_t u0 = hdr.y, u1 = hdr.z, u2 = hdr.w;
      const uint32_t s03 = u0 & 0x3f3f3f3fu, m03 = u1 & 0x3f3f3f3fu;
      const uint32_t s47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
      const uint32_t m47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
      const float d = h2f((uint16_t)(hdr.x & 0xFFFFu)), dmin = h2f((uint16_t)(hdr.x >> 16));
      h8 bq, c = {};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t sc = ((j < 4 ? s03 : s47) >> (8 * (j & 3))) & 0xFFu;
        const uint32_t mn = ((j < 4 ? m03 : m47) >> (8 * (j & 3))) & 0xFFu;
        bq[j] = (_Float16)((8.0f * d * (float)sc - dmin * (float)mn) * kToB);
      }
      const _Float16 d4 = (_Float16)(4.0f * d * kToB);  // exact: 4 d 2^8 of an f16 d
      c[0] = d4;
      c[1] = d4;
      *(h8*)&s_cop[n][0] = bq;
      *(h8*)&s_cop[n][8] = c;
      s_d4[n] = 4.0f * d;
    }
  };

  // ---- accumulators ----
  i16v T[2][2];
  f16v acc[2][2];
  i16v magic;
#pragma unroll
  for (int i = 0; i < 16; i++) magic[i] = (int)kMagic;
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc[a][c][i] = 0.0f;

  // the lane's operand rows within the staged tiles
  const int arow0 = 64 * wm + r32, arow1 = arow0 + 32;
  const int bcol0 = 64 * wn + r32, bcol1 = bcol0 + 32;
  // fragment lane offsets for K-step ks (rows 32 apart share a swizzle, and
  // the A and B rows of a lane share it too)
  uint32_t fa[4], fb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
    const uint32_t pc = 16u * ((uint32_t)(2 * ks + h) ^ swz((uint32_t)r32));
    fa[ks] = (uint32_t)arow0 * kStage + pc;
    fb[ks] = (uint32_t)bcol0 * kStage + pc;
  }
  // (fa[ks] = fa[0] ^ 32 ks: bits 5-6 of a row's offset are its swizzled
  // K-step; Q6_K forms them so at each use, which keeps 6 registers free)
  auto frag = [&](const int8_t* base, int t2, int ks, bool a_side) -> i4v {
    const uint32_t f = Q6 ? (a_side ? fa[0] : fb[0]) ^ (32u * (uint32_t)ks) : (a_side ? fa[ks] : fb[ks]);
    return lds_ld<i4v>(lds_addr(base) + f + 32u * kStage * (uint32_t)t2);
  };

  // ---- prologue: row factors, stage 0 ----
#pragma unroll
  for (int u = 0; u < 4; u++) dma_a1(2 * sb0, s_a0, u);
#pragma unroll
  for (int u = 0; u < F::kWaveCopies; u++) dma_w1(sb0, s_w0, u);
  dma_rows(sb0, 0);
  dma_rows(sb0, 1);
  // each split's row factors (the maximum over its own super-blocks, so a
  // split's result does not depend on the workgroup that computes it); 8
  // loads in flight at a time, and the maximum does not depend on the order
  // (fmaxf skips NaN)
  float rfp[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if (tid < 256) {
    const float* __restrict__ yr = yd + prow * nsb;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if (q >= P) break;
      const int e0 = sb0 + q * plen, e1 = e0 + (P == 1 ? sb1 - sb0 : plen);
      float mx = 0.0f;
      for (int sb = e0; sb < e1; sb += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = sb + j < e1 ? yr[sb + j] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[j]));
      }
      rfp[q] = row_factor(mx);
    }
    s_rf[tid] = rfp[0];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  build(s_w0, 0, s_b0, sb0);
  __syncthreads();

  // One stage: MFMAs on (sa, sbt); the next stage's weights expanded into
  // nbt from nw (half nhalf) and its activation copied into na; on the first
  // half of a super-block, the next super-block's raw weights copied into
  // wnext and this super-block's scales prepared from wcur; on the second
  // half, the epilogue.
  auto stage = [&](int sb, int half, const int8_t* sa, const int8_t* sbt, int8_t* na, int8_t* nbt,
                   const uint8_t* nw, int nhalf, const uint8_t* wcur, uint8_t* wnext) {
    const int g = 2 * sb + half;
    const bool more = g + 1 < 2 * sb1;
    const bool wmore = half == 0 && sb + 1 < sb1;  // the next super-block's raw weights
    const bool rmore = half == 1 && sb + 1 < sb1;  // the next super-block's row inputs
#pragma unroll
    for (int ks = 0; ks < (Q6 ? 1 : 4); ks++) {
      opaque(fa[ks]);
      opaque(fb[ks]);
    }
    opaque(x_raw);
    opaque(x_w0);
    if constexpr (!Q6) opaque(x_w1);
    i4v a0 = frag(sa, 0, 0, true), a1 = frag(sa, 1, 0, true);
    i4v b0 = frag(sbt, 0, 0, false), b1 = frag(sbt, 1, 0, false);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const bool first = half == 0 && ks == 0;
      T[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, first ? magic : T[0][0], 0, 0, 0);
      T[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, first ? magic : T[0][1], 0, 0, 0);
      T[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, first ? magic : T[1][0], 0, 0, 0);
      T[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, first ? magic : T[1][1], 0, 0, 0);
      // The next K-step's fragments into the same registers: an MFMA reads
      // its operands when it issues, so the reads overlap the four MFMAs
      // without a second register set.
      if (ks < 3) {
        a0 = frag(sa, 0, ks + 1, true);
        a1 = frag(sa, 1, ks + 1, true);
        b0 = frag(sbt, 0, ks + 1, false);
        b1 = frag(sbt, 1, ks + 1, false);
      }
      // this K-step's share of the next stage's copies
      if (more) dma_a1(g + 1, na, ks);
      if (wmore && ks < F::kWaveCopies) dma_w1(sb + 1, wnext, ks);
      if (rmore && ks < 2) dma_rows(sb + 1, ks);
      if (ks == 1 && more) build(nw, nhalf, nbt, (g + 1) >> 1);
    }
    if (half == 0) {
      prep(wcur, sb);
    } else {
      // epilogue of super-block sb: the f16 product (min term, offset, and
      // the magic correction), then acc += (1.5 2^23 + T) * 4 d dy
      h8 ra0, ra1, cb0, cb1;
      if constexpr (Q6) {
        // the magic correction only: A = dy_h (2^16, 2^15), B = -dq 2^7 (twice)
        const float y0 = h ? 0.0f : s_dy[arow0], y1 = h ? 0.0f : s_dy[arow1];
        const float q0 = h ? 0.0f : -128.0f * s_d4[bcol0], q1 = h ? 0.0f : -128.0f * s_d4[bcol1];
        ra0 = h8{(_Float16)(y0 * 65536.0f), (_Float16)(y0 * 32768.0f), 0, 0, 0, 0, 0, 0};
        ra1 = h8{(_Float16)(y1 * 65536.0f), (_Float16)(y1 * 32768.0f), 0, 0, 0, 0, 0, 0};
        cb0 = h8{(_Float16)q0, (_Float16)q0, 0, 0, 0, 0, 0, 0};
        cb1 = h8{(_Float16)q1, (_Float16)q1, 0, 0, 0, 0, 0, 0};
      } else {
        ra0 = *(const h8*)&s_rop[arow0][8 * h];
        ra1 = *(const h8*)&s_rop[arow1][8 * h];
        cb0 = *(const h8*)&s_cop[bcol0][8 * h];
        cb1 = *(const h8*)&s_cop[bcol1][8 * h];
      }
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ra0, cb0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ra0, cb1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ra1, cb0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ra1, cb1, acc[1][1], 0, 0, 0);
      const float d40 = s_d4[bcol0], d41 = s_d4[bcol1];
#pragma unroll
      for (int tm = 0; tm < 2; tm++) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const float4 dy4 = *(const float4*)&s_dy[64 * wm + 32 * tm + 8 * gq + 4 * h];
          const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            // the element by value: __builtin_bit_cast of a vector element
            // reads element 0 for every index (clang, ROCm 7.2)
            const int i = 4 * gq + e;
            const int t0 = T[tm][0][i], t1 = T[tm][1][i];
            acc[tm][0][i] = __builtin_fmaf(__int_as_float(t0), dyv[e] * d40, acc[tm][0][i]);
            acc[tm][1][i] = __builtin_fmaf(__int_as_float(t1), dyv[e] * d41, acc[tm][1][i]);
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  constexpr float kOutScale = Q6 ? 1.0f / 64.0f : 1.0f;  // Q6_K: its extra 1/2 and the 2^7 of dq
  const int tl = ct * mtiles + mt;  // the tile within its weight
  auto store_slot = [&](int sp) {
    float* __restrict__ mine = a.part + pick(a.part_off) + ((int64_t)tl * S + sp) * (kBM * kBN);
#pragma unroll
    for (int tn = 0; tn < 2; tn++)
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int lr = 64 * wm + 32 * tm + 8 * (i >> 2) + 4 * h + (i & 3);
          mine[(32 * tn + 16 * tm + i) * kThreads + tid] = acc[tm][tn][i] * inv_pow2(s_rf[lr]) * kOutScale;
        }
  };

  for (int sb = sb0; sb < sb1; sb += 2) {
    stage(sb, 0, s_a0, s_b0, s_a1, s_b1, s_w0, 1, s_w0, s_w1);
    stage(sb, 1, s_a1, s_b1, s_a0, s_b0, s_w1, 0, s_w0, s_w1);
    if (sb + 1 < sb1) {
      stage(sb + 1, 0, s_a0, s_b0, s_a1, s_b1, s_w1, 1, s_w1, s_w0);
      stage(sb + 1, 1, s_a1, s_b1, s_a0, s_b0, s_w0, 0, s_w1, s_w0);
    }
    if constexpr (!Q6) {
      // the end of a split that is not the workgroup's last: its partial to
      // its slot, the accumulators cleared, the next split's row factors
      const int q = (sb + 2 - sb0) / plen;
      if (P > 1 && sb + 2 < sb1 && sb + 2 - sb0 == q * plen) {
        store_slot(split + q - 1);
#pragma unroll
        for (int x = 0; x < 2; x++)
#pragma unroll
          for (int c = 0; c < 2; c++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[x][c][i] = 0.0f;
        __syncthreads();
        if (tid < 256) s_rf[tid] = q == 1 ? rfp[1] : q == 2 ? rfp[2] : rfp[3];
        __syncthreads();
      }
    }
  }

  // ---- store, the row factor undone (exact powers of two) ----
  float* __restrict__ dst = pick(a.dst);
  const int64_t ldd = pick(a.ldd);
  if (S == 1) {
#pragma unroll
    for (int tn = 0; tn < 2; tn++) {
      const int64_t col = n0 + 64 * wn + 32 * tn + r32;
      if (col >= N) continue;
#pragma unroll
      for (int tm = 0; tm < 2; tm++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int lr = 64 * wm + 32 * tm + 8 * (i >> 2) + 4 * h + (i & 3);
          const int64_t row = m0 + lr;
          if (row < M) dst[row * ldd + col] = acc[tm][tn][i] * inv_pow2(s_rf[lr]) * kOutScale;
        }
    }
    return;
  }
  // Several K splits: each writes its partial tile to its slot, in register
  // order (element e of thread tid at e * 512 + tid: every store a full line
  // per wave); gemm_q4k_sp_sum_kernel adds the slots in split order.
  store_slot(split + P - 1);
}

// dst of the split tiles: each thread adds, for 2 groups of 4 consecutive
// slot elements (4 neighbouring columns of one row), the splits' partials in
// split order ((p0 + p1) + p2) + p3, every slot's loads issued before the
// first add. Split tile b of the launch is weight t's tile b - tile_base[t];
// a workgroup covers 512 groups of one tile, so b, t and S are uniform.
constexpr int kSumThreads = 256;
constexpr int kSumBlocksPerTile = kBM * kBN / 4 / (2 * kSumThreads);  // 16
__global__ __launch_bounds__(kSumThreads) void gemm_q4k_sp_sum_kernel(const SpArgs a) {
  const int b = (int)blockIdx.x / kSumBlocksPerTile;
  const int t = b < a.tile_base[1] ? 0 : b < a.tile_base[2] ? 1 : b < a.tile_base[3] ? 2 : 3;
  auto pick = [&](const auto& arr) { return t == 0 ? arr[0] : t == 1 ? arr[1] : t == 2 ? arr[2] : arr[3]; };
  const int S = pick(a.splits);  // 2 or 4
  const int tl = b - pick(a.tile_base);
  const int mt = tl % a.mtiles, ct = tl / a.mtiles;
  const int64_t N = pick(a.n), ldd = pick(a.ldd), M = a.M;
  float* __restrict__ dbase = pick(a.dst);
  const bool vec = (ldd & 3) == 0 && ((uintptr_t)dbase & 15) == 0;
  const float* __restrict__ tile = a.part + pick(a.part_off) + (int64_t)tl * S * (kBM * kBN);
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int kSlot = kBM * kBN;
  int o[2];
  f4 v[2][4];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    // element offset in the slot: e * 512 + tid of the GEMM's register order
    o[j] = 4 * (((int)blockIdx.x % kSumBlocksPerTile) * (2 * kSumThreads) + j * kSumThreads + (int)threadIdx.x);
    v[j][0] = __builtin_nontemporal_load((const f4*)(tile + o[j]));
    v[j][1] = __builtin_nontemporal_load((const f4*)(tile + kSlot + o[j]));
  }
  if (S > 2) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      v[j][2] = __builtin_nontemporal_load((const f4*)(tile + 2 * kSlot + o[j]));
      v[j][3] = __builtin_nontemporal_load((const f4*)(tile + 3 * kSlot + o[j]));
    }
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    f4 sum = v[j][0] + v[j][1];
    if (S > 2) {
      sum += v[j][2];
      sum += v[j][3];
    }
    // the slot position of element 0: e = o / 512, thread tid = o % 512 (the 4 share e, wave and h)
    const int e = o[j] >> 9, tid = o[j] & 511, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 3, wn = wv >> 2, h = lane >> 5, r32 = lane & 31;
    const int tn = e >> 5, tm = (e >> 4) & 1, i = e & 15;
    const int64_t row = (int64_t)mt * kBM + 64 * wm + 32 * tm + 8 * (i >> 2) + 4 * h + (i & 3);
    const int64_t col = (int64_t)ct * kBN + 64 * wn + 32 * tn + r32;
    if (row >= M) continue;
    float* __restrict__ d = dbase + row * ldd + col;
    if (vec && col + 3 < N) {
      *(f4*)d = sum;
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (col + q < N) d[q] = sum[q];
    }
  }
}

}  // namespace

constexpr int64_t kSpMinK = 2048;

int gemm_q4k_sp_min_rows() { return 129; }

bool gemm_q4k_sp_fits(int64_t n, int64_t k, int64_t rows) {
  // The rounding of sc (q - 8) adds an error that shrinks as 1/sqrt(k)
  // relative to ||w|| ||x||: from k = 2048 it stays within half the 2e-3
  // bound; shorter rows keep the exact two-pass kernel. 32-bit byte offsets
  // inside the kernel.
  return k % 256 == 0 && k >= kSpMinK && n * (k / 256) * 144 < ((int64_t)1 << 31) &&
         (rows + kBM) * k < ((int64_t)1 << 31) && rows < ((int64_t)1 << 24);
}

// K splits of one weight's product: while its tiles fill at most half the
// CUs, the K range is cut in two (to 4), each part at least 4 super-blocks.
// Chosen per weight, so a weight's result does not depend on the weights it
// shares a launch with.
int gemm_q4k_sp_splits(int64_t n, int64_t k, int64_t rows, int cus) {
  const int64_t nsb = k / 256;
  const int64_t tiles = ((rows + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  int S = 1;
  while (S < 4 && tiles * S * 2 <= cus && nsb % (2 * S) == 0 && nsb / (2 * S) >= 4) S *= 2;
  return S;
}

static size_t split_slot_bytes(int64_t n, int64_t rows, int S) {
  return S > 1 ? (size_t)(((rows + kBM - 1) / kBM) * ((n + kBN - 1) / kBN)) * S * kBM * kBN * 4 : 0;
}
static size_t split_tiles(int64_t n, int64_t rows, int S) {
  return S > 1 ? (size_t)(((rows + kBM - 1) / kBM) * ((n + kBN - 1) / kBN)) : 0;
}

size_t gemm_q4k_sp_split_bytes(const MvTargets& t, int64_t k, int64_t rows, int cus) {
  size_t slots = 0, tiles = 0;
  int64_t prev = 0;
  for (int i = 0; i < t.count; i++) {
    const int64_t n = t.row_end[i] - prev;
    prev = t.row_end[i];
    const int S = gemm_q4k_sp_splits(n, k, rows, cus);
    slots += split_slot_bytes(n, rows, S);
    tiles += split_tiles(n, rows, S);
  }
  (void)tiles;
  return slots;
}

template <int FMT>
hipError_t launch_sp(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, void* split_ws, size_t split_bytes,
                     int cus, hipStream_t st) {
  if (t.count < 1 || t.count > kMaxTargets) return hipErrorInvalidValue;
  const size_t need = gemm_q4k_sp_split_bytes(t, k, rows, cus);
  const bool split = need > 0 && split_ws != nullptr && split_bytes >= need;
  SpArgs a{};
  a.yq = p.codes;
  a.yd = p.d;
  a.ybs = (const int16_t*)p.sums;
  a.M = rows;
  a.nsb = (int)(k / 256);
  a.mtiles = (int)((rows + kBM - 1) / kBM);
  // K splits per weight (from its own shape), then, where the launch's
  // workgroups exceed the CUs (several weights), Q4_K workgroups that
  // compute 2 or 4 consecutive splits of a tile: the same partial tiles, so
  // the same bits, in one round of workgroups
  int S_[kMaxTargets], P_[kMaxTargets];
  int64_t wt_[kMaxTargets];
  for (int i = 0; i < t.count; i++) {
    const int64_t n = t.row_end[i] - (i ? t.row_end[i - 1] : 0);
    S_[i] = split ? gemm_q4k_sp_splits(n, k, rows, cus) : 1;
    P_[i] = 1;
    wt_[i] = (int64_t)a.mtiles * ((n + kBN - 1) / kBN);
  }
  if (FMT == T_Q4_K) {
    for (;;) {
      int64_t total = 0;
      int best = -1;
      for (int i = 0; i < t.count; i++) {
        const int64_t u = wt_[i] * (S_[i] / P_[i]);
        total += u;
        if (S_[i] / P_[i] >= 2 && (best < 0 || u > wt_[best] * (S_[best] / P_[best]))) best = i;
      }
      if (total <= cus || best < 0) break;
      P_[best] *= 2;
    }
  }
  int64_t units = 0, slot_floats = 0;
  int tiles = 0;
  for (int i = 0; i < kMaxTargets; i++) {
    const int j = i < t.count ? i : t.count - 1;  // unused entries repeat the last weight, with no units
    const int64_t n = t.row_end[j] - (j ? t.row_end[j - 1] : 0);
    a.w[i] = t.w[j];
    a.dst[i] = t.dst[j];
    a.ldd[i] = t.ldd[j];
    a.n[i] = n;
    a.splits[i] = S_[j];
    a.per[i] = P_[j];
    a.tile_base[i] = tiles;
    a.part_off[i] = slot_floats;
    if (i < t.count) {
      units += wt_[i] * (S_[i] / P_[i]);
      if (S_[i] > 1) {
        tiles += (int)wt_[i];
        slot_floats += wt_[i] * S_[i] * kBM * kBN;
      }
    }
    a.unit_end[i] = (int)units;
  }
  if (units >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  a.remap = units % 8 == 0 ? 1 : 0;
  a.part = tiles > 0 ? (float*)split_ws : nullptr;
  gemm_kq_sp_kernel<FMT><<<dim3((unsigned)units), kThreads, 0, st>>>(a);
  if (tiles > 0) {
    // unused entries past the last weight start at the end (no workgroups)
    for (int i = t.count; i < kMaxTargets; i++) a.tile_base[i] = tiles;
    gemm_q4k_sp_sum_kernel<<<dim3((unsigned)(tiles * kSumBlocksPerTile)), kSumThreads, 0, st>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_q4k_sp_targets(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, void* split_ws,
                                      size_t split_bytes, int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  return launch_sp<T_Q4_K>(t, k, p, rows, split_ws, split_bytes, cus, st);
}

hipError_t launch_gemm_q6k_sp_targets(const MvTargets& t, int64_t k, const ActPlanes& p, int64_t rows, void* split_ws,
                                      size_t split_bytes, int cus, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  return launch_sp<T_Q6_K>(t, k, p, rows, split_ws, split_bytes, cus, st);
}

bool gemm_q6k_sp_fits(int64_t n, int64_t k, int64_t rows) {
  // rows 16-byte aligned (210 (k / 256) a multiple of 16) and the single
  // pass's rounding small against ||w|| ||x|| (k >= 2048, as for Q4_K)
  return k % 2048 == 0 && n * (k / 256) * 210 < ((int64_t)1 << 31) && (rows + kBM) * k < ((int64_t)1 << 31) &&
         rows < ((int64_t)1 << 24);
}

hipError_t launch_gemm_q6k_sp(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                              int64_t ldd, hipStream_t st) {
  MvTargets t{};
  t.w[0] = w;
  t.dst[0] = dst;
  t.ldd[0] = ldd;
  t.row_end[0] = n;
  t.count = 1;
  return launch_gemm_q6k_sp_targets(t, k, p, rows, nullptr, 0, 256, st);
}

hipError_t launch_gemm_q4k_sp(const void* w, int64_t n, int64_t k, const ActPlanes& p, int64_t rows, float* dst,
                              int64_t ldd, hipStream_t st) {
  MvTargets t{};
  t.w[0] = w;
  t.dst[0] = dst;
  t.ldd[0] = ldd;
  t.row_end[0] = n;
  t.count = 1;
  return launch_gemm_q4k_sp_targets(t, k, p, rows, nullptr, 0, 256, st);
}

}  // namespace qmm
