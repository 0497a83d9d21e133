// mv_common.h — pieces the streaming decode kernels share (internal to
// libqmm): the activation's home in LDS, filled by the workgroup either by
// quantizing f32 rows (Q8_K, bit-exact to BlockQ8K::from_float,
// vendor/candle/candle-core/src/quantized/k_quants.rs:2882-2927) or by
// copying pre-quantized planes; and the staging of byte spans of a weight
// row through LDS for formats whose blocks are not 16-byte aligned.
#pragma once

#include "qmm_device.h"

#include <mutex>
#include "qmm_launch.h"

namespace qmm {

// The activation in LDS: codes int8 [NR][k], d f32 [NR][nsb], and the sum of
// the codes of each group of 16 values int32 [NR][nsb*16] (the reference's
// bsums).
struct ActLds {
  int8_t* codes;
  float* dy;
  int32_t* s16;
};

__host__ __device__ inline size_t act_lds_bytes(int nr, int nsb) {
  const size_t a = (size_t)nr * nsb * 256;
  const size_t b = (a + (size_t)nr * nsb * 4 + 15) / 16 * 16;
  return b + (size_t)nr * nsb * 64;
}

__device__ __forceinline__ ActLds act_lds(uint8_t* base, int nr, int nsb) {
  const size_t a = (size_t)nr * nsb * 256;
  const size_t b = (a + (size_t)nr * nsb * 4 + 15) / 16 * 16;
  ActLds s;
  s.codes = (int8_t*)base;
  s.dy = (float*)(base + a);
  s.s16 = (int32_t*)(base + b);
  return s;
}

// The activation part of LDS: FUSED quantizes the f32 rows, else copies
// pre-quantized planes. A pass of a wave covers four Q8_K blocks, one per
// group of 16 lanes (lane gl of a group holds values 16gl..16gl+15 of its
// block); pass p of wave w covers blocks 4(p*kWaves + w) .. +3 of the
// NR x nsb blocks. The loads of the first kPasses passes are issued before
// the weight loads (ActBatch::load) so that waiting for them does not mean
// waiting for HBM; further passes load and store one after another.
constexpr int kPasses = 2;

template <int NR, bool FUSED, int kWaves>
struct ActBatch {
  uint4 v[kPasses][4];  // FUSED: 16 f32 values; else [0] = 16 codes, [1].x = d bits, [1].y = sum of the 16

  __device__ __forceinline__ static int block_of(int pass, int wv) {
    return (pass * kWaves + wv) * 4 + ((threadIdx.x & 63) >> 4);
  }

  __device__ __forceinline__ static void load_pass(uint4 (&v)[4], int b, int nsb, const float* __restrict__ x,
                                                   int64_t xstride, const int8_t* __restrict__ yq,
                                                   const float* __restrict__ yd, const int16_t* __restrict__ ybs) {
    const int gl = threadIdx.x & 15;
    if (b >= NR * nsb) return;
    const int r = b / nsb, sb = b - r * nsb;
    if (FUSED) {
      // rows 16-byte aligned (the launcher checks x and xstride)
      const uint4* xp = (const uint4*)(x + r * xstride + sb * 256 + 16 * gl);
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = xp[i];
    } else {
      const int k = nsb * 256;
      v[0] = *(const uint4*)(yq + (int64_t)r * k + sb * 256 + 16 * gl);
      v[1].x = __float_as_uint(yd[r * nsb + sb]);
      v[1].y = (uint32_t)(int32_t)ybs[(r * nsb + sb) * 16 + gl];
    }
  }

  __device__ __forceinline__ void load(int nsb, const float* x, int64_t xstride, const int8_t* yq, const float* yd,
                                       const int16_t* ybs) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int p = 0; p < kPasses; p++) {
#pragma unroll
      for (int i = 0; i < 4; i++) v[p][i] = make_uint4(0, 0, 0, 0);
      if ((p * kWaves + wv) * 4 < NR * nsb) load_pass(v[p], block_of(p, wv), nsb, x, xstride, yq, yd, ybs);
    }
  }

  // every lane of the wave calls (the quantizer's shuffles span the groups)
  __device__ __forceinline__ static void store_pass(const ActLds& s, const uint4 (&v)[4], int b, int nsb, float qmax) {
    const int gl = threadIdx.x & 15;
    uint32_t c[4];
    int32_t sum16;
    float d;
    if (FUSED) {
      float f[16];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        f[4 * i] = __uint_as_float(v[i].x); f[4 * i + 1] = __uint_as_float(v[i].y);
        f[4 * i + 2] = __uint_as_float(v[i].z); f[4 * i + 3] = __uint_as_float(v[i].w);
      }
      q8k_block_group16(f, gl, qmax, c, sum16, d);
    } else {
      c[0] = v[0].x; c[1] = v[0].y; c[2] = v[0].z; c[3] = v[0].w;
      d = __uint_as_float(v[1].x);
      sum16 = (int32_t)v[1].y;
    }
    if (b >= NR * nsb) return;
    const int k = nsb * 256;
    const int r = b / nsb, sb = b - r * nsb;
    *(uint4*)(s.codes + r * k + sb * 256 + 16 * gl) = make_uint4(c[0], c[1], c[2], c[3]);
    s.s16[(r * nsb + sb) * 16 + gl] = sum16;
    if (gl == 0) s.dy[r * nsb + sb] = d;
  }

  __device__ __forceinline__ void store(const ActLds& s, int nsb, const float* x, int64_t xstride, const int8_t* yq,
                                        const float* yd, const int16_t* ybs, float qmax) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int p = 0; p < kPasses; p++)
      if ((p * kWaves + wv) * 4 < NR * nsb) store_pass(s, v[p], block_of(p, wv), nsb, qmax);
    for (int p = kPasses; (p * kWaves + wv) * 4 < NR * nsb; p++) {
      uint4 t[4] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
      load_pass(t, block_of(p, wv), nsb, x, xstride, yq, yd, ybs);
      store_pass(s, t, block_of(p, wv), nsb, qmax);
    }
  }
};

// The same fill with a Q8_K block per wave pass (lane L: values 4L..4L+3,
// q8k_block_wave): every wave of the workgroup has a block while the blocks
// are at least as many as the waves, and each lane's dependent chain is four
// values long. Pass p of wave w covers block p * kWaves + w.
template <int NR, bool FUSED, int kWaves, int kPre>
struct ActBatchW {
  uint4 v[kPre];  // FUSED: 4 f32 values; else .x = 4 codes, .y = d bits, .z = the quad's sum

  __device__ __forceinline__ static void load_pass(uint4& v, int b, int nsb, const float* __restrict__ x,
                                                   int64_t xstride, const int8_t* __restrict__ yq,
                                                   const float* __restrict__ yd, const int16_t* __restrict__ ybs) {
    const int lane = threadIdx.x & 63;
    v = make_uint4(0, 0, 0, 0);
    if (b >= NR * nsb) return;
    const int r = b / nsb, sb = b - r * nsb;
    if (FUSED) {
      v = *(const uint4*)(x + r * xstride + sb * 256 + 4 * lane);  // rows 16-byte aligned
    } else {
      const int k = nsb * 256;
      v.x = *(const uint32_t*)(yq + (int64_t)r * k + sb * 256 + 4 * lane);
      v.y = __float_as_uint(yd[r * nsb + sb]);
      v.z = (uint32_t)(int32_t)ybs[(r * nsb + sb) * 16 + (lane >> 2)];
    }
  }

  __device__ __forceinline__ static void store_pass(const ActLds& s, const uint4& v, int b, int nsb, float qmax) {
    const int lane = threadIdx.x & 63;
    uint32_t c;
    int32_t sum16;
    float d;
    if (FUSED) {
      const float f[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
      q8k_block_wave(f, lane, qmax, c, sum16, d);
    } else {
      c = v.x;
      d = __uint_as_float(v.y);
      sum16 = (int32_t)v.z;
    }
    if (b >= NR * nsb) return;
    const int k = nsb * 256;
    const int r = b / nsb, sb = b - r * nsb;
    *(uint32_t*)(s.codes + r * k + sb * 256 + 4 * lane) = c;
    if ((lane & 3) == 0) s.s16[(r * nsb + sb) * 16 + (lane >> 2)] = sum16;
    if (lane == 0) s.dy[r * nsb + sb] = d;
  }

  __device__ __forceinline__ void load(int nsb, const float* x, int64_t xstride, const int8_t* yq, const float* yd,
                                       const int16_t* ybs) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int p = 0; p < kPre; p++) load_pass(v[p], p * kWaves + wv, nsb, x, xstride, yq, yd, ybs);
  }

  __device__ __forceinline__ void store(const ActLds& s, int nsb, const float* x, int64_t xstride, const int8_t* yq,
                                        const float* yd, const int16_t* ybs, float qmax) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int p = 0; p < kPre; p++)
      if (p * kWaves + wv < NR * nsb) store_pass(s, v[p], p * kWaves + wv, nsb, qmax);
    for (int p = kPre; p * kWaves + wv < NR * nsb; p++) {
      uint4 t;
      load_pass(t, p * kWaves + wv, nsb, x, xstride, yq, yd, ybs);
      store_pass(s, t, p * kWaves + wv, nsb, qmax);
    }
  }
};

// ---------------------------------------------------------------------------
// LDS staging for formats whose blocks are not 16-byte aligned. A wave
// copies a span of a weight row (4096 values) into its own LDS region with
// linear 16-byte loads from the 16-byte boundary at or before the span's
// first byte. Every 16-byte piece read holds at least one byte of the row,
// and a 16-byte aligned piece never crosses a page, so the over-read at
// either end stays inside mapped memory.
// ---------------------------------------------------------------------------
constexpr int kSpanMaxBytes = 4352;                  // 128 Q8_0 blocks, the largest span
constexpr int kStageBytes = kSpanMaxBytes + 16 + 16; // + alignment slack + over-read

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Copies bytes [start, start+len) of W into lds; returns the LDS offset of `start`.
__device__ __forceinline__ int stage_span(const uint8_t* __restrict__ W, int64_t start, int len, uint8_t* lds,
                                          int lane) {
  const int64_t a0 = start & ~(int64_t)15;
  const int pieces = (int)((start + len - a0 + 15) >> 4);
  for (int p = lane; p < pieces; p += 64) *(uint4*)(lds + 16 * p) = *(const uint4*)(W + a0 + 16 * p);
  return (int)(start - a0);
}

// 4 bytes from LDS at any byte offset (two aligned dword reads + alignbyte;
// the hardware takes unaligned LDS reads too, but measured slower).
__device__ __forceinline__ uint32_t lds_u32(const uint8_t* lds, int off) {
  const int a = off & ~3;
  const uint32_t lo = *(const uint32_t*)(lds + a);
  const uint32_t hi = *(const uint32_t*)(lds + a + 4);
  return __builtin_amdgcn_alignbyte(hi, lo, (uint32_t)(off & 3));
}
// n consecutive dwords from LDS at any byte offset.
template <int N>
__device__ __forceinline__ void lds_words(const uint8_t* lds, int off, uint32_t* out) {
  const int a = off & ~3;
  const uint32_t s = (uint32_t)(off & 3);
  uint32_t w[N + 1];
#pragma unroll
  for (int i = 0; i <= N; i++) w[i] = *(const uint32_t*)(lds + a + 4 * i);
#pragma unroll
  for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], s);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* lds, int off) { return lds_u32(lds, off) & 0xFFFF; }

// ---------------------------------------------------------------------------
// Q6_K spans: a super-block is 210 bytes, so blocks are not 16-byte aligned;
// a wave stages a span of up to 16 super-blocks of a row in its own LDS
// buffer and each lane reads its unit from there.
// ---------------------------------------------------------------------------
constexpr int kQ6SpanSb = 16;                            // super-blocks per span
constexpr int kQ6SpanBytes = kQ6SpanSb * 210;              // 3360
constexpr int kQ6SpanPieces = (kQ6SpanBytes + 15) / 16 + 1; // 16-byte pieces, start not aligned: 211
constexpr int kQ6PiecesPerLane = (kQ6SpanPieces + 63) / 64; // 4
// LDS bytes per wave: the pieces, and the 8 bytes past the last that the
// dword reads of lds_words may touch
constexpr int kQ6SpanBuf = kQ6SpanPieces * 16 + 16;

struct Q6Span {
  uint4 p[kQ6PiecesPerLane];
  int off;  // offset of the span's first byte in its first piece
  int len;  // super-blocks in the span
};

// Loads the 16-byte aligned pieces (aligned as device addresses) from the one
// holding byte p to the one holding byte p + len*210 - 1. Every piece read
// holds at least one byte of the span, and an aligned piece never crosses a
// page, so the bytes read beyond the span stay in mapped memory. Lane L holds
// pieces L + 64c.
__device__ __forceinline__ void load_q6_span(Q6Span& sp, const uint8_t* __restrict__ p, int len, int lane) {
  // rounded down by pointer arithmetic: the compiler keeps these global
  // loads (an integer round trip would make them flat loads, which every LDS
  // wait also waits for)
  sp.off = (int)((uintptr_t)p & 15);
  const uint8_t* a0 = p - sp.off;
  sp.len = len;
  const int pieces = (int)((sp.off + len * 210 + 15) >> 4);
  // every lane loads (no branches): lanes past the span's pieces load its
  // last piece again, whose bytes are never read
#pragma unroll
  for (int c = 0; c < kQ6PiecesPerLane; c++) {
    const int pc = lane + 64 * c;
    sp.p[c] = ld_stream16(a0 + 16u * (uint32_t)(pc < pieces ? pc : pieces - 1));
  }
}

// A lane's operands of one Q6_K unit (q6k_unit) from a span staged in LDS: the
// super-block at LDS offset b, half h, l0 = 0 or 16.
struct Q6Lane {
  uint32_t qlA[4], qlB[4], qh[4];
  int sc[4];
  float dx;
};

__device__ __forceinline__ void load_q6_lane(const uint8_t* buf, int b, int h, int l0, Q6Lane& u) {
  uint32_t s4[2];
  lds_words<4>(buf, b + 64 * h + l0, u.qlA);
  lds_words<4>(buf, b + 64 * h + 32 + l0, u.qlB);
  lds_words<4>(buf, b + 128 + 32 * h + l0, u.qh);
  lds_words<2>(buf, b + 192 + 8 * h, s4);  // scales 8h .. 8h+7
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int gg = (l0 >> 4) + 2 * t;
    u.sc[t] = (int)(int8_t)((s4[gg >> 2] >> (8 * (gg & 3))) & 0xFF);
  }
  u.dx = h2f((uint16_t)lds_u16(buf, b + 208));
}

// Dynamic LDS past 64 KiB needs the kernel's limit raised (to the 160 KiB of
// a CU), once per kernel function and device (raise_lds_limit, qmm_api.hip).
// Each launcher names its kernel as a template argument, which registers the
// kernel when the library loads (big_lds_register), so qmm_prepare can raise
// every such limit before a capture begins.
bool big_lds_register(const void* fn);
hipError_t raise_lds_limit(const void* fn);
template <auto F>
struct BigLds {
  static const bool registered;
};
template <auto F>
const bool BigLds<F>::registered = big_lds_register((const void*)F);

template <auto F>
inline hipError_t set_max_dynamic_lds() {
  (void)BigLds<F>::registered;
  return raise_lds_limit((const void*)F);
}

}  // namespace qmm
