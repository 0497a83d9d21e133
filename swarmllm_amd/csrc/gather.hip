// gather.hip — rows of a quantized table picked by id (the embedding lookup
// of a GGUF token table), bytes copied whole: QTensor::gather_rows
// (vendor/candle/candle-core/src/quantized/mod.rs:1039-1091) and
// QCudaStorage::gather_rows (quantized/cuda.rs:1478-1540), which runs
// candle's index_select over the bytes (candle-kernels/src/indexing.cu:41-69).
//
// A row is hidden / block_size blocks of the table's type, so it starts on a
// block boundary and its bytes are copied unchanged: the output holds the
// same GGUF blocks as the chosen rows and dequantizes to the same values.
// One workgroup per output row (grid-stride over rows), its threads copying
// the row in 16-, 4- or 1-byte units, whichever the row size and the two
// buffers' alignment allow.
//
// Ids: u32. An id of 0xFFFFFFFF writes a zero row, as index_select does for
// the index type's maximum (indexing.cu:60-61); a row of zero bytes
// dequantizes to zeros in every block format here. Any other id past the
// vocabulary writes a zero row too, and is counted into *bad when the
// caller passes a counter: the reference's host path refuses such an id
// (mod.rs:1075-1077) and its device path asserts (indexing.cu:63), and a
// kernel here neither traps nor aborts, so the caller reads the count.
#include <hip/hip_runtime.h>

#include "../../include/qmm.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace qmm {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kNoRow = 0xFFFFFFFFu;

template <typename U>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const U* __restrict__ table, int64_t vocab,
                                                               int64_t units, const uint32_t* __restrict__ ids,
                                                               int64_t n_ids, U* __restrict__ out,
                                                               uint32_t* __restrict__ bad) {
  for (int64_t r = blockIdx.x; r < n_ids; r += gridDim.x) {
    const uint32_t id = ids[r];
    const bool ok = (int64_t)id < vocab && id != kNoRow;
    U* __restrict__ dst = out + r * units;
    if (ok) {
      const U* __restrict__ src = table + (int64_t)id * units;
      for (int64_t u = threadIdx.x; u < units; u += kThreads) dst[u] = src[u];
    } else {
      for (int64_t u = threadIdx.x; u < units; u += kThreads) dst[u] = U{};
      if (threadIdx.x == 0 && id != kNoRow && bad != nullptr) atomicAdd(bad, 1u);
    }
  }
}

// block size and block bytes of the types a table may hold: the five
// product formats and the plain F32 / F16 / BF16 a GGUF keeps beside them
bool table_type(int type, int64_t& bs, int64_t& ts) {
  switch (type) {
    case 0: bs = 1; ts = 4; return true;     // F32
    case 1: bs = 1; ts = 2; return true;     // F16
    case 30: bs = 1; ts = 2; return true;    // BF16
    case T_Q8_0: bs = 32; ts = 34; return true;
    case T_IQ4_NL: bs = 32; ts = 18; return true;
    case T_MXFP4: bs = 32; ts = 17; return true;
    case T_Q4_K: bs = 256; ts = 144; return true;
    case T_Q6_K: bs = 256; ts = 210; return true;
    default: return false;
  }
}

template <typename U>
hipError_t launch_gather(const void* table, int64_t vocab, int64_t row_bytes, const uint32_t* ids, int64_t n_ids,
                         void* out, uint32_t* bad, hipStream_t st) {
  QMM_NOTE_LAUNCH();
  const int64_t grid = n_ids < 65536 ? n_ids : 65536;
  gather_rows_kernel<U><<<dim3((unsigned)grid), kThreads, 0, st>>>((const U*)table, vocab,
                                                                    row_bytes / (int64_t)sizeof(U), ids, n_ids,
                                                                    (U*)out, bad);
  return hipGetLastError();
}

}  // namespace
}  // namespace qmm

extern "C" {

int qmm_gather_row_bytes(int type, int64_t hidden, size_t* row_bytes) {
  int64_t bs = 0, ts = 0;
  if (!row_bytes || !qmm::table_type(type, bs, ts) || hidden <= 0 || hidden % bs) return QMM_UNSUPPORTED;
  *row_bytes = (size_t)(hidden / bs * ts);
  return QMM_OK;
}

int qmm_gather_rows(int type, const void* table, size_t table_bytes, int64_t vocab, int64_t hidden,
                    const uint32_t* ids, int64_t n_ids, void* out, size_t out_bytes, uint32_t* bad,
                    int64_t stream) {
  size_t rb = 0;
  if (qmm_gather_row_bytes(type, hidden, &rb) != QMM_OK) return QMM_UNSUPPORTED;
  if (vocab <= 0 || n_ids < 0 || vocab > ((int64_t)1 << 40) || n_ids > ((int64_t)1 << 40)) return QMM_UNSUPPORTED;
  const int64_t row_bytes = (int64_t)rb;
  if (vocab > INT64_MAX / row_bytes || n_ids > INT64_MAX / row_bytes) return QMM_UNSUPPORTED;
  if (table == nullptr || table_bytes < (size_t)(vocab * row_bytes)) return QMM_UNSUPPORTED;
  if (out_bytes < (size_t)(n_ids * row_bytes)) return QMM_WORKSPACE_TOO_SMALL;
  if (n_ids == 0) return QMM_OK;
  if (ids == nullptr || out == nullptr) return QMM_UNSUPPORTED;
  (void)hipGetLastError();
  const hipStream_t st = (hipStream_t)stream;
  const uintptr_t al = (uintptr_t)table | (uintptr_t)out | (uintptr_t)row_bytes;
  hipError_t e;
  if ((al & 15) == 0)
    e = qmm::launch_gather<uint4>(table, vocab, row_bytes, ids, n_ids, out, bad, st);
  else if ((al & 3) == 0)
    e = qmm::launch_gather<uint32_t>(table, vocab, row_bytes, ids, n_ids, out, bad, st);
  else
    e = qmm::launch_gather<uint8_t>(table, vocab, row_bytes, ids, n_ids, out, bad, st);
  return e == hipSuccess ? QMM_OK : QMM_DEVICE_ERROR;
}

}  // extern "C"
