// glu_act.h — the gated activations of an MLP's gate and up products,
// act(gate) * up, shared by the fused gate+up+GLU decode kernel and the
// elementwise kernel, so both give the same bits for the same inputs.
//
// The expressions of the reference's fused ops (src/inference/fast_math.rs):
//   SiLU       gate / (1 + exp(-gate)) * up                         (:48-60)
//   SwigluOai  x = min(gate, 7) (a NaN gate stays NaN),
//              y = clamp(up, -7, 7) (a NaN up stays NaN),
//              x / (1 + exp(1.702 * -x)) * (y + 1)                  (:84-104)
//   GELU       0.5 v (1 + tanh(0.7978846 v (1 + 0.044715 v v))) * up, the
//              tanh form of candle's f32 gelu                        (:62-76)
// Device exp and tanh are not the host's libm: results agree with the
// reference within a few units in the last place, not bit for bit.
#pragma once

#include <hip/hip_runtime.h>

namespace qmm {

enum GluAct : int { GLU_SILU = 0, GLU_SWIGLU_OAI = 1, GLU_GELU = 2 };

constexpr float kSwigluOaiAlpha = 1.702f;
constexpr float kSwigluOaiLimit = 7.0f;
constexpr float kGeluSqrtTwoOverPi = 0.7978846f;

// No contraction into fma: every caller rounds each operation alike.
template <int ACT>
__device__ __forceinline__ float glu_act(float g, float u) {
#pragma clang fp contract(off)
  if constexpr (ACT == GLU_SILU) {
    return g / (1.0f + expf(-g)) * u;
  } else if constexpr (ACT == GLU_SWIGLU_OAI) {
    const float x = kSwigluOaiLimit < g ? kSwigluOaiLimit : g;
    const float y = u < -kSwigluOaiLimit ? -kSwigluOaiLimit : (u > kSwigluOaiLimit ? kSwigluOaiLimit : u);
    return x / (1.0f + expf(kSwigluOaiAlpha * (-x))) * (y + 1.0f);
  } else {
    const float a = 0.5f * g * (1.0f + tanhf(kGeluSqrtTwoOverPi * g * (1.0f + 0.044715f * g * g)));
    return a * u;
  }
}

}  // namespace qmm
