// b32_common.h — the 32-value block formats (Q8_0, IQ4_NL, MXFP4) read from
// LDS, and the per-unit arithmetic every kernel over them shares (the decode
// matvec and the grouped expert products), so a product's bits do not depend
// on which kernel ran it.
#pragma once

#include "mv_common.h"

namespace qmm {

// 16-entry int8 table lookup of the 4 nibbles at bit sh (0 or 4) of the
// bytes of n. Entries 0-7 (t0, t1) and 8-15 (t2, t3) are each looked up by
// the nibble's low 3 bits, and a third byte permute takes byte i from the
// first (selector i) or, where the nibble's bit 3 is set, from the second
// (selector i + 4): six or seven instructions for 4 values. The selector is
// one v_and_or_b32 (the compiler otherwise splits it into an and and an or
// with literal operands, which a three-operand instruction cannot take on
// gfx9); its two constants come in registers, the mask a scalar one.
__device__ __forceinline__ int32_t lut16_at(uint32_t n, int sh, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t v = n >> sh;
  const uint32_t sel = v & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
  uint32_t pick;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(pick) : "v"(v >> 1), "s"(0x04040404u), "v"(0x03020100u));
  return (int32_t)__builtin_amdgcn_perm(hi, lo, pick);
}

__device__ __forceinline__ uint32_t pack4(const int8_t* t) {
  return (uint32_t)(uint8_t)t[0] | ((uint32_t)(uint8_t)t[1] << 8) | ((uint32_t)(uint8_t)t[2] << 16) |
         ((uint32_t)(uint8_t)t[3] << 24);
}

// Block decode from LDS at byte offset off: 32 int8 weights in q (value i of
// the block in byte i%4 of word i/4) and the f32 block scale d. For MXFP4 and
// IQ4_NL the values are the format's table entries (k_quants.rs:30-54: the
// E2M1 table doubled to integers with the e8m0 scale halved to match;
// IQ4NL_VALUES), low nibbles first.
template <int FMT>
struct Fmt32;
template <>
struct Fmt32<T_Q8_0> {
  static constexpr int B = 34;
  __device__ static void decode(const uint8_t* L, int off, uint32_t q[8], float& d, uint32_t, uint32_t, uint32_t,
                                uint32_t) {
    d = h2f((uint16_t)lds_u16(L, off));
    lds_words<8>(L, off + 2, q);
  }
};
template <>
struct Fmt32<T_IQ4_NL> {
  static constexpr int B = 18;
  __device__ static void decode(const uint8_t* L, int off, uint32_t q[8], float& d, uint32_t t0, uint32_t t1,
                                uint32_t t2, uint32_t t3) {
    d = h2f((uint16_t)lds_u16(L, off));
    uint32_t n[4];
    lds_words<4>(L, off + 2, n);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      q[i] = (uint32_t)lut16_at(n[i], 0, t0, t1, t2, t3);
      q[4 + i] = (uint32_t)lut16_at(n[i], 4, t0, t1, t2, t3);
    }
  }
};
template <>
struct Fmt32<T_MXFP4> {
  static constexpr int B = 17;
  __device__ static void decode(const uint8_t* L, int off, uint32_t q[8], float& d, uint32_t t0, uint32_t t1,
                                uint32_t t2, uint32_t t3) {
    d = e8m0_half(lds_u32(L, off) & 0xFF);
    uint32_t n[4];
    lds_words<4>(L, off + 1, n);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      q[i] = (uint32_t)lut16_at(n[i], 0, t0, t1, t2, t3);
      q[4 + i] = (uint32_t)lut16_at(n[i], 4, t0, t1, t2, t3);
    }
  }
};

// The lookup table of a format, packed for lut16_at.
template <int FMT>
struct Lut32 {
  uint32_t t0, t1, t2, t3;
  __device__ Lut32() {
    const int8_t* tab = FMT == T_MXFP4 ? kMxfp4Values : kIq4nlValues;
    t0 = pack4(tab);
    t1 = pack4(tab + 4);
    t2 = pack4(tab + 8);
    t3 = pack4(tab + 12);
  }
};

// A lane's 64 activation values (two blocks) of one row: codes and scales.
struct Act64 {
  int y[2][8];
  float dy[2];
};

// Loads the codes and scales of blocks gb, gb+1 of activation row `row`
// (Q8_0 planes: codes [rows][k], scales [rows][k/32]); `two` = block gb+1
// exists.
__device__ __forceinline__ void load_act64(Act64& a, const int8_t* __restrict__ yq, const float* __restrict__ yd,
                                           int64_t row, int64_t k, int nb, int64_t gb, bool two) {
  const int8_t* yrow = yq + row * k + gb * 32;
  const int4 a0 = *(const int4*)yrow;
  const int4 b0 = *(const int4*)(yrow + 16);
  a.y[0][0] = a0.x; a.y[0][1] = a0.y; a.y[0][2] = a0.z; a.y[0][3] = a0.w;
  a.y[0][4] = b0.x; a.y[0][5] = b0.y; a.y[0][6] = b0.z; a.y[0][7] = b0.w;
  a.dy[0] = yd[row * nb + gb];
  if (two) {
    const int4 a1 = *(const int4*)(yrow + 32);
    const int4 b1 = *(const int4*)(yrow + 48);
    a.y[1][0] = a1.x; a.y[1][1] = a1.y; a.y[1][2] = a1.z; a.y[1][3] = a1.w;
    a.y[1][4] = b1.x; a.y[1][5] = b1.y; a.y[1][6] = b1.z; a.y[1][7] = b1.w;
    a.dy[1] = yd[row * nb + gb + 1];
  } else {
#pragma unroll
    for (int t = 0; t < 8; t++) a.y[1][t] = 0;
    a.dy[1] = 0.0f;
  }
}

// acc + the unit's two block dots: (dx0 dy0) s0 + (dx1 dy1) s1 with exact
// int32 block sums s and every f32 operation rounded on its own, none
// contracted into an fma (the block
// dot of candle's vec_dot per type: Q8_0 k_quants.rs:1294-1312, MXFP4
// :517-527, IQ4_NL :754-764).
__device__ __forceinline__ float b32_unit(const uint32_t q0[8], const uint32_t q1[8], float dx0, float dx1,
                                          const Act64& a, float acc) {
#pragma clang fp contract(off)
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    s0 = dot4((int)q0[t], a.y[0][t], s0);
    s1 = dot4((int)q1[t], a.y[1][t], s1);
  }
  // plain operators: the pragma governs only the operations written here
  // (__fmul_rn and __fadd_rn are ordinary * and + in functions of their own,
  // which the compiler may still fuse once inlined)
  const float p0 = (dx0 * a.dy[0]) * (float)s0;
  const float p1 = (dx1 * a.dy[1]) * (float)s1;
  return acc + (p0 + p1);
}

}  // namespace qmm
