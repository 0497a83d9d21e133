// qmm_noalloc.hip — qmm_forward for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc): the activation scratch qmm_forward takes as a workspace
// argument lives in a file-scope device array instead.
//
// Each GPU the library runs on holds its own copy of `scratch` (16 MiB) until
// the process ends. Host code never names the array as a device address: its
// per-device address comes from hipGetSymbolAddress, looked up once per
// device on the first call with that device current, and only that address
// reaches kernels. Every call on a device shares the array, which keeps the
// last call's contents; calls that overlap on one device (two streams, two
// threads) race on it. The kernels overwrite every byte they read back, so
// nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/qmm.h"

namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, or nullptr when the
// lookup failed (the failure is reported to the caller as a device error).
void* scratch_on_current_device() {
  static std::mutex mu;
  static void* ptr[kMaxDevices];
  static bool looked_up[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!looked_up[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;  // not cached: a later call retries the lookup
    }
    ptr[dev] = p;
    looked_up[dev] = true;
  }
  return ptr[dev];
}

}  // namespace

namespace qmm {
// The scratch's address on the current device looked up ahead of a first
// call (qmm_prepare): false when the lookup failed.
bool noalloc_prepare() { return scratch_on_current_device() != nullptr; }
}  // namespace qmm

extern "C" {

size_t qmm_forward_noalloc_max_bytes(void) { return kScratchBytes; }

int qmm_forward_noalloc(int type, const void* w, const float* x, int64_t x_stride, float* dst, int64_t ldd,
                        int64_t k, int64_t n, int64_t rows, int64_t stream) {
  size_t need = 0;
  const int plan = qmm_forward(type, w, x, x_stride, dst, ldd, nullptr, 0, &need, k, n, rows, 0, stream);
  if (plan != QMM_OK) return plan;
  // `need` may count a GEMM's K-split slots, which it goes without when the
  // scratch holds only the quantized activation
  const size_t least = qmm_act_bytes(qmm_act_layout(type, rows), k, rows);
  if (need > kScratchBytes && least > kScratchBytes) return QMM_WORKSPACE_TOO_SMALL;  // nothing enqueued
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return QMM_DEVICE_ERROR;
  return qmm_forward(type, w, x, x_stride, dst, ldd, ws, kScratchBytes, &need, k, n, rows, 1, stream);
}

}  // extern "C"
