// wire.hip — the Q8_0 hidden-state wire codec: the bytes a layer split sends
// between the peers that hold consecutive layers
// (src/inference/quant.rs:1-107, quantize_q8_0 / dequantize_q8_0).
//
// Per 32 values: [f16 scale][32 x i8] = 34 bytes, a partial trailing group
// zero-padded. The block maximum skips non-finite values; scale = amax / 127
// (f32), the codes clamp(round(v * (1 / scale)), -127, 127) with the
// reciprocal of the unrounded f32 scale; the scale travels as f16 (round to
// nearest even) and decoding multiplies by that f16 value. Built without FP
// contraction: the codes are the reference's bit for bit.
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

// Largest of 32 lanes (the half-wave's own), through DPP within rows of 16
// and one swap of the row halves.
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad 1,0,3,2
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));   // quad 2,3,0,1
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));  // half mirror
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // mirror
  // rows of 16 hold their maximum in every lane; the other row of this half-wave
  const int lane = (int)(threadIdx.x & 63);
  const float o = __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, __float_as_int(v)));
  return fmaxf(v, o);
}

// Rust's `f32 as i8` after f32::clamp(-127, 127): NaN -> 0.
__device__ __forceinline__ int8_t wire_code(float v, float inv) {
  const float qf = roundf(v * inv);  // f32::round: half away from zero
  if (qf != qf) return 0;
  return (int8_t)(qf < -127.0f ? -127.0f : (qf > 127.0f ? 127.0f : qf));
}

__global__ __launch_bounds__(256) void wire_encode_kernel(const float* __restrict__ x, int64_t n,
                                                          uint8_t* __restrict__ out) {
  const int64_t blk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  const int lane = (int)(threadIdx.x & 31);
  const int64_t nb = (n + 31) / 32;
  const bool live = blk < nb;  // every lane of a half-wave takes part in the reductions
  const int64_t i = blk * 32 + lane;
  const bool valid = live && i < n;
  const float v = valid ? x[i] : 0.0f;
  const float a = __builtin_isfinite(v) ? fabsf(v) : 0.0f;
  const float amax = half_wave_max(a);
  const float scale = amax == 0.0f ? 0.0f : amax / 127.0f;
  const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  if (!live) return;
  uint8_t* b = out + blk * 34;
  b[2 + lane] = (uint8_t)(valid ? wire_code(v, inv) : 0);
  if (lane == 0) {
    const uint16_t h = f2h(scale);
    b[0] = (uint8_t)(h & 0xFF);
    b[1] = (uint8_t)(h >> 8);
  }
}

__global__ __launch_bounds__(256) void wire_decode_kernel(const uint8_t* __restrict__ in, int64_t n,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint8_t* b = in + (i >> 5) * 34;
  const float scale = h2f((uint16_t)(b[0] | (b[1] << 8)));
  out[i] = (float)(int8_t)b[2 + (i & 31)] * scale;
}

}  // namespace

int64_t wire_bytes(int64_t n) {
  if (n < 0) return -1;
  const int64_t blocks = n / 32 + (n % 32 != 0);
  if (blocks > INT64_MAX / 34) return -1;
  return blocks * 34;
}

hipError_t launch_wire_encode(const float* x, int64_t n, void* out, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t threads = (n + 31) / 32 * 32;
  wire_encode_kernel<<<dim3((unsigned)((threads + 255) / 256)), 256, 0, st>>>(x, n, (uint8_t*)out);
  return hipGetLastError();
}

hipError_t launch_wire_decode(const void* in, int64_t n, float* out, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  wire_decode_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, st>>>((const uint8_t*)in, n, out);
  return hipGetLastError();
}

}  // namespace qmm
