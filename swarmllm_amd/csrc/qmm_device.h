// qmm_device.h — device-side layouts and helpers shared by the HIP kernels
// of libqmm (gfx950 / CDNA4, wave64).
//
// Block layouts are the GGUF ones (byte-identical to candle's repr(C)
// structs, vendor/candle/candle-core/src/quantized/k_quants.rs:165-317):
// weights stay in the bytes a GGUF file holds, so a QTensor's data() is
// the device buffer as is.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

constexpr int kWave = 64;

// GGUF type ids (vendor/candle/candle-core/src/quantized/mod.rs:319-371).
enum : int {
  T_Q8_0 = 8,
  T_Q4_K = 12,
  T_Q6_K = 14,
  T_Q8_K = 15,
  T_IQ4_NL = 20,
  T_MXFP4 = 39,
};

struct blk_q8_0 { uint16_t d; int8_t qs[32]; };                                     // 34 B / 32
struct blk_q4_k { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };          // 144 B / 256
struct blk_q6_k { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; }; // 210 B / 256
struct blk_q8_k { float d; int8_t qs[256]; int16_t bsums[16]; };                     // 292 B / 256
struct blk_mxfp4 { uint8_t e; uint8_t qs[16]; };                                     // 17 B / 32
struct blk_iq4_nl { uint16_t d; uint8_t qs[16]; };                                   // 18 B / 32
static_assert(sizeof(blk_q8_0) == 34, "q8_0");
static_assert(sizeof(blk_q4_k) == 144, "q4_k");
static_assert(sizeof(blk_q6_k) == 210, "q6_k");
static_assert(sizeof(blk_q8_k) == 292, "q8_k");
static_assert(sizeof(blk_mxfp4) == 17, "mxfp4");
static_assert(sizeof(blk_iq4_nl) == 18, "iq4_nl");

// Values of a 4-bit code: k_quants.rs:30-36.
__device__ __constant__ static const int8_t kIq4nlValues[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                                                1, 13, 25, 38, 53, 69, 89, 113};
__device__ __constant__ static const int8_t kMxfp4Values[16] = {0, 1, 2, 3, 4, 6, 8, 12,
                                                                0, -1, -2, -3, -4, -6, -8, -12};

// ---- f16 <-> f32 (IEEE binary16, round to nearest even; f16 denormals kept)
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// A 16-byte load of weight bytes a product reads once, each byte by exactly
// one load: the nontemporal hint streams them past the caches (measured ~10%
// more HBM throughput for contiguous pieces on gfx950). Loads that share
// cache lines must not use it: each would fetch the line again.
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const v4u t = __builtin_nontemporal_load((const v4u*)p);
  return make_uint4(t.x, t.y, t.z, t.w);
}
// f32 -> f16 in integer arithmetic. A plain (_Float16) cast of a product may
// be folded into a mixed-precision multiply-add with +0, which turns -0 into
// +0; the conversion here is the IEEE one for every input, signed zeros and
// subnormal halves included.
__device__ __forceinline__ uint16_t f2h(float f) {
  const uint32_t x = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t e8 = (x >> 23) & 0xFFu;
  const uint32_t m23 = x & 0x7FFFFFu;
  if (e8 == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m23 ? (0x200u | (m23 >> 13)) : 0u));
  const int e = (int)e8 - 112;  // biased half exponent
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m = m23 | 0x800000u;
    const int shift = 14 - e;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (m23 >> 13);
  const uint32_t rem = m23 & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;  // a carry into the exponent is correct
  return (uint16_t)(sign | h);
}

// Half an E8M0 scale, exactly: 2^(e-128), subnormal below e = 2 (k_quants.rs:39-54).
__device__ __forceinline__ float e8m0_half(uint32_t e) {
  const uint32_t bits = e < 2 ? (0x00200000u << e) : ((e - 1u) << 23);
  return __builtin_bit_cast(float, bits);
}

// ---- Rust conversions: truncate toward zero, saturate, NaN -> 0 ----------
__device__ __forceinline__ int32_t rs_as_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return 2147483647;
  if (v <= -2147483648.0f) return (-2147483647 - 1);
  return (int32_t)v;
}
__device__ __forceinline__ int32_t rs_as_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int32_t)v;
}
__device__ __forceinline__ uint32_t rs_as_u8(float v) {
  if (v != v) return 0;
  if (v >= 255.0f) return 255;
  if (v <= 0.0f) return 0;
  return (uint32_t)v;
}
// f32::max / f32::min: the non-NaN operand wins; between equals the second.
__device__ __forceinline__ float rs_max(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  return a > b ? a : b;
}
__device__ __forceinline__ float rs_min(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  return a < b ? a : b;
}
// nearest_int (k_quants utils.rs:1): round half away from zero, then as i32.
__device__ __forceinline__ int32_t nearest_int(float v) { return rs_as_i32(roundf(v)); }
__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// ---- wave64 reductions ----------------------------------------------------
// Sum over the 64 lanes: DPP within rows of 16, then the four row sums, in a
// fixed order (every decode kernel of a format reduces with this one, so a
// row's result does not depend on which kernel or batch width computed it).
// The sums of the four 16-lane rows of the wave (DPP within each row).
__device__ __forceinline__ void wave_row16_sums(float v, float& a, float& b, float& c, float& d) {
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad 1,0,3,2
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));   // quad 2,3,0,1
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));  // half mirror
  v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // mirror
  a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  float a, b, c, d;
  wave_row16_sums(v, a, b, c, d);
  return __fadd_rn(__fadd_rn(a, b), __fadd_rn(c, d));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// ---- activation quantizer -------------------------------------------------
// One Q8_K code (BlockQ8K::from_float, k_quants.rs:2917-2920): the reference
// computes t = iscale * x, then t.round() (half away from zero), .min(127.)
// (which gives 127 for NaN) and `as i8` (saturating). For every float t that
// equals trunc(clamp(t + copysign(0.49999997, t), -128.49, 127.49)): adding
// the float just below one half reaches the next integer exactly when t is at
// or above the tie (round to nearest even resolves the one boundary case,
// 0.49999997 + 0.5, upwards), and the clamp, taken with min first, sends NaN
// to 127 and the infinities (a denormal block maximum can make iscale
// infinite) to the saturated codes. Checked against the reference's steps for
// all 2^32 floats (tests/test_act_rounding.py restates the check on the
// half-integer neighbourhoods). Four instructions and the conversion.
__device__ __forceinline__ int32_t q8k_code(float t) {
#pragma clang fp contract(off)
  const float s = t + __builtin_copysignf(0.49999997f, t);
  return (int32_t)fmaxf(fminf(s, 127.49f), -128.49f);
}

// One Q8_0 code (BlockQ8_0::from_float, k_quants.rs:1262-1265): the
// reference computes t = x * id, then t.round() (half away from zero) and
// `as i8` (saturating, NaN gives 0). The same rounding as q8k_code, then
// v_cvt_i32_f32 (which truncates, saturates out-of-range values and gives 0
// for NaN) and a clamp to -128..127. Checked against the reference's steps
// for all 2^32 floats (tests/act_rounding_exhaustive.c).
__device__ __forceinline__ int32_t cvt_i32_trunc_sat(float f) {
  int32_t r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
  return r;
}
__device__ __forceinline__ int32_t q8_0_code(float t) {
#pragma clang fp contract(off)
  const int32_t q = cvt_i32_trunc_sat(t + __builtin_copysignf(0.49999997f, t));
  return q < -128 ? -128 : (q > 127 ? 127 : q);
}

// 4 codes (each in -128..127) packed one per byte, code 0 in the low byte.
__device__ __forceinline__ uint32_t pack4_i8(int32_t a, int32_t b, int32_t c, int32_t d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0C0C0400u);  // a.b0, b.b0, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000C0Cu);  // 0, 0, c.b0, d.b0
  return lo | hi;
}

// Maximum over the lane's row of 16 (DPP: pairs, pairs of pairs, then the
// mirrored halves and rows); every lane of the row gets the result.
template <int CTL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t row16_maxu(uint32_t k) {
  k = max(k, dpp_u<0xB1>(k));
  k = max(k, dpp_u<0x4E>(k));
  k = max(k, dpp_u<0x141>(k));
  return max(k, dpp_u<0x140>(k));
}

// The reference's block scale value is the signed value of the FIRST element
// of largest |x| (strict <; NaN never qualifies, as `amax < |x|` is false for
// it). With p the largest of 0 and the values and m the largest of 0 and the
// negated values (fmaxf ignores NaN, so neither is NaN and both are >= 0,
// ordered as their bits), |max| = max(p, m) and its sign is p's or n's unless
// p == m != 0, where both signs reach it and the first such element decides:
// that rare case takes the maximum of the key (0xFFFF - index, sign), the
// lowest index. The key's base is made opaque inside the branch so that the
// compiler does not keep the per-value keys live outside it.

// Q8_K of one 256-value block held by a group of 16 lanes (gl = lane within
// the group, 0..15), lane gl holding values 16gl..16gl+15 in v[0..15].
// Returns the lane's 16 codes packed in c[0..3], their sum (the reference's
// bsums entry gl) and d. All 64 lanes must call.
__device__ __forceinline__ void q8k_block_group16(const float v[16], int gl, float qmax, uint32_t c[4],
                                                  int32_t& sum16, float& d) {
#pragma clang fp contract(off)
  float p = 0.0f, m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    p = fmaxf(p, v[i]);
    m = fmaxf(m, -v[i]);
  }
  const uint32_t pb = row16_maxu(__float_as_uint(p)), mb = row16_maxu(__float_as_uint(m));
  const float amax = __uint_as_float(max(pb, mb));
  sum16 = 0;
  d = 0.0f;
  c[0] = c[1] = c[2] = c[3] = 0u;
  if (amax != 0.0f) {
    float mx = pb > mb ? amax : -amax;
    if (pb == mb) {
      uint32_t base = (uint32_t)(0xFFFF - 16 * gl) << 1;
      asm volatile("" : "+v"(base));
      uint32_t key = 0;
#pragma unroll
      for (int i = 15; i >= 0; i--)
        if (fabsf(v[i]) == amax) key = (base - 2u * (uint32_t)i) | (__float_as_uint(v[i]) >> 31);
      key = row16_maxu(key);
      mx = (key & 1u) ? -amax : amax;
    }
    const float iscale = -qmax / mx;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      int32_t q[4];
#pragma unroll
      for (int e = 0; e < 4; e++) q[e] = q8k_code(iscale * v[4 * w + e]);
      c[w] = pack4_i8(q[0], q[1], q[2], q[3]);
      sum16 = __builtin_amdgcn_sdot4((int)c[w], 0x01010101, sum16, false);
    }
    d = 1.0f / iscale;
  }
}

// The same Q8_K block held by a whole wave: lane L holds values 4L..4L+3 in
// v[0..3]. The maxima are taken within each row of 16 lanes (DPP), then over
// the four rows (readlane, uniform). Returns the lane's 4 codes packed in c,
// the sum of the 16 values of the lane's quad (lanes 4g..4g+3: the
// reference's bsums entry g) in sum16, and d. All 64 lanes must call.
__device__ __forceinline__ void q8k_block_wave(const float v[4], int lane, float qmax, uint32_t& c, int32_t& sum16,
                                               float& d) {
#pragma clang fp contract(off)
  const float p = fmaxf(fmaxf(0.0f, v[0]), fmaxf(v[1], fmaxf(v[2], v[3])));
  const float m = fmaxf(fmaxf(0.0f, -v[0]), fmaxf(-v[1], fmaxf(-v[2], -v[3])));
  uint32_t pr = row16_maxu(__float_as_uint(p)), mr = row16_maxu(__float_as_uint(m));
  uint32_t pb = (uint32_t)__builtin_amdgcn_readlane((int)pr, 0), mb = (uint32_t)__builtin_amdgcn_readlane((int)mr, 0);
#pragma unroll
  for (int r = 1; r < 4; r++) {
    pb = max(pb, (uint32_t)__builtin_amdgcn_readlane((int)pr, 16 * r));
    mb = max(mb, (uint32_t)__builtin_amdgcn_readlane((int)mr, 16 * r));
  }
  const float amax = __uint_as_float(max(pb, mb));
  c = 0u;
  int32_t s = 0;
  d = 0.0f;
  if (amax != 0.0f) {
    float mx = pb > mb ? amax : -amax;
    if (pb == mb) {
      uint32_t base = (uint32_t)(0xFFFF - 4 * lane) << 1;
      asm volatile("" : "+v"(base));
      uint32_t key = 0;
#pragma unroll
      for (int i = 3; i >= 0; i--)
        if (fabsf(v[i]) == amax) key = (base - 2u * (uint32_t)i) | (__float_as_uint(v[i]) >> 31);
      key = row16_maxu(key);
      uint32_t kb = (uint32_t)__builtin_amdgcn_readlane((int)key, 0);
#pragma unroll
      for (int r = 1; r < 4; r++) kb = max(kb, (uint32_t)__builtin_amdgcn_readlane((int)key, 16 * r));
      mx = (kb & 1u) ? -amax : amax;
    }
    const float iscale = -qmax / mx;
    c = pack4_i8(q8k_code(iscale * v[0]), q8k_code(iscale * v[1]), q8k_code(iscale * v[2]), q8k_code(iscale * v[3]));
    s = __builtin_amdgcn_sdot4((int)c, 0x01010101, 0, false);
    d = 1.0f / iscale;
  }
  s += __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, true);
  s += __builtin_amdgcn_mov_dpp(s, 0x4E, 0xF, 0xF, true);
  sum16 = s;
}

// Q4_K 6-bit scale/min of sub-block j (k_quants utils.rs:50-60).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& d, int& m) {
  if (j < 4) {
    d = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__device__ __forceinline__ int32_t dot4(int32_t a, int32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// One 64-value unit of a Q4_K x Q8_K product (k_quants.rs:2031-2111): chunk
// j (sub-blocks 2j, 2j+1) of a super-block with header h (d, dmin, scales)
// and code bytes qa, qb (qs[32j .. 32j+31]), against the activation's 64
// codes y (values 64j .. 64j+63 of the block), its d (dy) and the code sums
// of the two sub-blocks (p0, p1). Adds dy*(d*sum_sc - dmin*sum_m) to acc with
// every f32 operation rounded explicitly (the products and the difference on
// their own, the last step one fma), so each decode kernel that calls it gets
// the same bits for a unit.
__device__ __forceinline__ float q4k_unit(uint4 h, uint4 qa, uint4 qb, const int y[16], float dy, int32_t p0,
                                          int32_t p1, int j, float acc) {
#pragma clang fp contract(off)
  const int sh = 16 * (j & 1);
  const uint32_t u0 = h.y, u1 = h.z, u2 = h.w;
  const uint32_t scw = j < 2 ? (u0 & 0x3f3f3f3fu) : ((u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4));
  const uint32_t mw = j < 2 ? (u1 & 0x3f3f3f3fu) : (((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4));
  const int sc0 = (int)((scw >> sh) & 0xFF), sc1 = (int)((scw >> (sh + 8)) & 0xFF);
  const int m0 = (int)((mw >> sh) & 0xFF), m1 = (int)((mw >> (sh + 8)) & 0xFF);
  const float dx = h2f((uint16_t)(h.x & 0xFFFF));
  const float mx = h2f((uint16_t)(h.x >> 16));
  const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  int slo = 0, shi = 0;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    slo = dot4((int)(w[q] & 0x0F0F0F0Fu), y[q], slo);
    shi = dot4((int)((w[q] >> 4) & 0x0F0F0F0Fu), y[8 + q], shi);
  }
  // |slo|, |shi| <= 16*15*127 and |p| <= 32*127: 24-bit products are exact
  const float main = dx * (float)(__mul24(sc0, slo) + __mul24(sc1, shi));
  const float mins = mx * (float)(__mul24(m0, p0) + __mul24(m1, p1));
  return __builtin_fmaf(dy, main - mins, acc);
}

// One 64-value unit of a Q6_K x Q8_K product (k_quants.rs:2598-2655): half
// h of a super-block, values 128h + 32t + l0 + [0,16) for t = 0..3 (l0 = 0
// or 16). qlA = ql[64h + l0 ..], qlB = ql[64h + 32 + l0 ..], qh = qh[32h + l0 ..]
// (16 bytes each, as 4 words), sc[t] = scales[8h + l0/16 + 2t], dx = d;
// y[t] = the activation codes of group t, bs[t] their sum, dy the
// activation block's d. Adds (dx*dy) * sum_t sc_t * sum (q-32)*y to acc with
// every f32 operation rounded explicitly, so each decode kernel that calls it
// gets the same bits for a unit.
__device__ __forceinline__ float q6k_unit(const uint32_t qlA[4], const uint32_t qlB[4], const uint32_t qh[4],
                                          const int sc[4], float dx, const int y[4][4], float dy, const int bs[4],
                                          float acc) {
  // q6 = (ql nibble) | (qh bits 2t, 2t+1) << 4 for every byte, the high bits
  // taken where they already sit, shifted by 4 - 2t
  int sums[4] = {0, 0, 0, 0};
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t h = qh[q];
    const uint32_t q0 = (qlA[q] & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    const uint32_t q1 = (qlB[q] & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    const uint32_t q2 = ((qlA[q] >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    const uint32_t q3 = ((qlB[q] >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    sums[0] = dot4((int)q0, y[0][q], sums[0]);
    sums[1] = dot4((int)q1, y[1][q], sums[1]);
    sums[2] = dot4((int)q2, y[2][q], sums[2]);
    sums[3] = dot4((int)q3, y[3][q], sums[3]);
  }
  int tot = 0;
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int s = sums[t];
    // |s - 32*bs| <= 16*63*127 + 32*16*127 < 2^23: a 24-bit product is exact
    tot += __mul24(sc[t], s - 32 * bs[t]);
  }
  return __fmaf_rn(__fmul_rn(dx, dy), (float)tot, acc);
}

}  // namespace qmm
