// read_floor.hip — the bare streaming read a product's weight bytes are
// measured against: one launch that reads up to two spans of device memory
// once and does nothing else with them (a measurement aid, no counterpart in
// the reference).
//
// 1024 workgroups of 512 threads walk the spans in 16-byte nontemporal loads,
// lane-contiguous (a workgroup step covers 8 KB), one load of a lane at a
// time (the waves of a CU keep the requests in flight); each workgroup writes
// one word (the XOR of what it read) so the loads cannot be dropped. This is
// the fastest plain read shape of a sweep on MI355X over rotating 33 MB
// buffers (6.11 us a launch back to back; two, four or eight loads of a lane
// in flight 6.55-6.97 us, 2048 or 4096 workgroups 6.32-6.35 us, a contiguous
// block a workgroup 6.33-6.74 us); a matvec that reads the same bytes is held
// against its duration.
#include <hip/hip_runtime.h>

#include "../../include/qmm.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {
namespace {

constexpr int kThreads = 512, kBlocks = 1024, kDepth = 1;

__global__ __launch_bounds__(kThreads) void read_kernel(const uint4* __restrict__ a, int64_t na,
                                                        const uint4* __restrict__ b, int64_t nb,
                                                        uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t step = (int64_t)kBlocks * kThreads;
  const int64_t base = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (int s = 0; s < 2; s++) {
    const uint4* __restrict__ p = s == 0 ? a : b;
    const int64_t n = s == 0 ? na : nb;
    for (int64_t i = base; i < n; i += kDepth * step) {
      uint4 v[kDepth];
#pragma unroll
      for (int d = 0; d < kDepth; d++) {
        const int64_t e = i + d * step;
        v[d] = e < n ? ld_stream16(p + e) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int d = 0; d < kDepth; d++) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
  }
  __shared__ uint32_t red[kThreads / 64];
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kThreads / 64; w++) t ^= red[w];
    sink[blockIdx.x] = t;
  }
}

}  // namespace
}  // namespace qmm

extern "C" {

size_t qmm_read_floor_sink_bytes(void) { return (size_t)qmm::kBlocks * 4; }

int qmm_read_floor(const void* a, size_t a_bytes, const void* b, size_t b_bytes, void* sink, int64_t stream) {
  if ((a_bytes && !a) || (b_bytes && !b) || !sink || a_bytes % 16 || b_bytes % 16 || ((uintptr_t)a & 15) ||
      ((uintptr_t)b & 15))
    return QMM_UNSUPPORTED;
  (void)hipGetLastError();
  QMM_NOTE_LAUNCH();
  qmm::read_kernel<<<qmm::kBlocks, qmm::kThreads, 0, (hipStream_t)stream>>>(
      (const uint4*)a, (int64_t)(a_bytes / 16), (const uint4*)b, (int64_t)(b_bytes / 16), (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? QMM_OK : QMM_DEVICE_ERROR;
}

}  // extern "C"
