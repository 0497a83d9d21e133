// glu.hip — out = act(gate) * up elementwise, over rows of n values: the
// GLU between an MLP's gate and up products where they did not run as one
// fused launch (the reference's silu_mul / swiglu_oai_mul / gelu product,
// src/inference/fast_math.rs:48-130). The arithmetic is glu_act.h's, the
// fused decode kernel's.
#include "glu_act.h"
#include "qmm_launch.h"

namespace qmm {

namespace {

template <int ACT>
__global__ __launch_bounds__(256) void glu_kernel(const float* __restrict__ gate, int64_t ldg,
                                                  const float* __restrict__ up, int64_t ldu, float* __restrict__ out,
                                                  int64_t ldo, int64_t n, int64_t rows) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * rows) return;
  const int64_t r = i / n, c = i - r * n;
  out[r * ldo + c] = glu_act<ACT>(gate[r * ldg + c], up[r * ldu + c]);
}

template <int ACT>
hipError_t launch(const float* gate, int64_t ldg, const float* up, int64_t ldu, float* out, int64_t ldo, int64_t n,
                  int64_t rows, hipStream_t st) {
  const int64_t total = n * rows;
  if ((total + 255) / 256 >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  glu_kernel<ACT><<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(gate, ldg, up, ldu, out, ldo, n, rows);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_glu(int act, const float* gate, int64_t ldg, const float* up, int64_t ldu, float* out, int64_t ldo,
                      int64_t n, int64_t rows, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  if (n <= 0 || rows <= 0) return hipSuccess;
  if (act == GLU_SILU) return launch<GLU_SILU>(gate, ldg, up, ldu, out, ldo, n, rows, st);
  if (act == GLU_SWIGLU_OAI) return launch<GLU_SWIGLU_OAI>(gate, ldg, up, ldu, out, ldo, n, rows, st);
  if (act == GLU_GELU) return launch<GLU_GELU>(gate, ldg, up, ldu, out, ldo, n, rows, st);
  return hipErrorInvalidValue;
}

}  // namespace qmm
