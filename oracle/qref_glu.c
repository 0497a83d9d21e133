/* qref_glu.c — CPU oracle (test infrastructure only) of the gated
 * activations between an MLP's gate and up products, act(gate) * up, as the
 * reference's CPU path evaluates them (src/inference/fast_math.rs), in f32
 * with the host's libm (glibc) exp and tanh and no fused multiply-adds.
 *
 *   qref_silu_mul       gate / (1 + exp(-gate)) * up            (fast_math.rs:48-60, the scalar
 *                        form; its AVX2 form swaps libm's exp for a Cephes polynomial within 2 ulp)
 *   qref_swiglu_oai_mul min(gate, 7) (NaN stays NaN), clamp(up, -7, 7), x / (1 + exp(1.702 * -x)) * (y + 1)
 *                                                               (fast_math.rs:84-104)
 *   qref_gelu_mul       0.5 v (1 + tanh(0.7978846 v (1 + 0.044715 v v))) * up   (fast_math.rs:62-76)
 */
#include <math.h>
#include <stdint.h>

#include "qref.h"

void qref_silu_mul(const float *gate, const float *up, float *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    const float g = gate[i];
    out[i] = g / (1.0f + expf(-g)) * up[i];
  }
}

void qref_swiglu_oai_mul(const float *gate, const float *up, float *out, int64_t n) {
  const float limit = 7.0f, alpha = 1.702f;
  for (int64_t i = 0; i < n; i++) {
    const float g = gate[i], u = up[i];
    const float x = limit < g ? limit : g;
    const float y = u < -limit ? -limit : (u > limit ? limit : u);
    const float glu = x / (1.0f + expf(alpha * (-x)));
    out[i] = glu * (y + 1.0f);
  }
}

void qref_gelu_mul(const float *gate, const float *up, float *out, int64_t n) {
  const float c = 0.7978846f;
  for (int64_t i = 0; i < n; i++) {
    const float v = gate[i];
    const float g = 0.5f * v * (1.0f + tanhf(c * v * (1.0f + 0.044715f * v * v)));
    out[i] = g * up[i];
  }
}
