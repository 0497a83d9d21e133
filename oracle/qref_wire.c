/*
 * qref_wire.c — CPU restatement of SwarmLLM's Q8_0 hidden-state wire codec
 * (src/inference/quant.rs:1-107), the format activations cross between the
 * peers of a layer split in. TEST INFRASTRUCTURE ONLY (the checker of the
 * HIP codec); see qref.h.
 *
 * Per 32 values: [f16 scale][32 x i8] = 34 bytes, a partial trailing group
 * zero-padded. Unlike candle's BlockQ8_0::from_float, the block maximum
 * skips non-finite values, the codes are clamped to [-127, 127] after
 * rounding, and the reciprocal is taken of the unrounded f32 scale.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "qref.h"

int64_t qref_wire_bytes(int64_t n) {
  /* q8_0_byte_len_checked (quant.rs:98-104): ceil(n / 32) * 34, or -1 when
   * the product would not fit */
  if (n < 0) return -1;
  const int64_t blocks = n / 32 + (n % 32 != 0);
  if (blocks > INT64_MAX / 34) return -1;
  return blocks * 34;
}

/* Rust's `f32 as i8`: truncate toward zero, saturate, NaN -> 0. */
static int8_t rs_as_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v;
}

/* quantize_q8_0 (quant.rs:24-60) */
void qref_wire_encode(const float *values, int64_t n, uint8_t *out) {
  const int64_t blocks = n / 32 + (n % 32 != 0);
  for (int64_t b = 0; b < blocks; b++) {
    const int64_t start = 32 * b;
    const int64_t len = n - start < 32 ? n - start : 32;
    const float *chunk = values + start;
    float amax = 0.0f;
    for (int64_t i = 0; i < len; i++) {
      const float v = chunk[i];
      if (isfinite(v)) {
        const float a = fabsf(v);
        if (a > amax) amax = a;
      }
    }
    const float scale = amax == 0.0f ? 0.0f : amax / 127.0f;
    const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
    uint8_t *blk = out + 34 * b;
    const uint16_t h = qref_f32_to_f16(scale);
    memcpy(blk, &h, 2); /* to_le_bytes */
    for (int lane = 0; lane < 32; lane++) {
      int8_t q = 0;
      if (lane < len) {
        const float qf = roundf(chunk[lane] * inv); /* f32::round: half away from zero */
        /* f32::clamp(-127, 127): NaN stays NaN (then `as i8` gives 0) */
        const float c = qf != qf ? qf : (qf < -127.0f ? -127.0f : (qf > 127.0f ? 127.0f : qf));
        q = rs_as_i8(c);
      }
      blk[2 + lane] = (uint8_t)q;
    }
  }
}

/* dequantize_q8_0 (quant.rs:65-92): 0, or -1 on a length mismatch */
int qref_wire_decode(const uint8_t *bytes, int64_t nbytes, int64_t n, float *out) {
  if (nbytes != qref_wire_bytes(n)) return -1;
  const int64_t blocks = n / 32 + (n % 32 != 0);
  int64_t written = 0;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t *blk = bytes + 34 * b;
    uint16_t h;
    memcpy(&h, blk, 2);
    const float scale = qref_f16_to_f32(h);
    const int64_t take = n - written < 32 ? n - written : 32;
    for (int64_t i = 0; i < take; i++) out[written + i] = (float)(int8_t)blk[2 + i] * scale;
    written += take;
  }
  return 0;
}
