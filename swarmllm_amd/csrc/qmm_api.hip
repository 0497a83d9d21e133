// qmm_api.hip — the C ABI of include/qmm.h: argument checks, the choice of
// kernel by activation rows (QCudaStorage::fwd's policy,
// vendor/candle/candle-core/src/quantized/cuda.rs:1653-1680, decided anew
// for MI355X), status codes, launch counters and host-side fault injection.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>
#include <utility>
#include <vector>

#include "../../include/qmm.h"
#include "qmm_device.h"
#include "qmm_launch.h"

namespace {

std::atomic<uint64_t> g_matvec_launches{0};
std::atomic<uint64_t> g_gemm_launches{0};
std::atomic<bool> g_fail_next{false};
std::atomic<uint64_t> g_moe_launches{0};
std::atomic<uint64_t> g_moe_prefill_launches{0};
// set_force_dmmv (quantized/cuda.rs:29-33): products of qmm_forward and its
// shared / GLU forms dequantize the weight against the f32 activation.
std::atomic<bool> g_force_dmmv{false};

int block_size(int type) {
  switch (type) {
    case qmm::T_Q8_0: case qmm::T_IQ4_NL: case qmm::T_MXFP4: return 32;
    case qmm::T_Q4_K: case qmm::T_Q6_K: return 256;
    default: return 0;
  }
}
int type_size(int type) {
  switch (type) {
    case qmm::T_Q8_0: return 34;
    case qmm::T_IQ4_NL: return 18;
    case qmm::T_MXFP4: return 17;
    case qmm::T_Q4_K: return 144;
    case qmm::T_Q6_K: return 210;
    default: return 0;
  }
}

// SWARMLLM_Q8K_SCALE=128: candle's Q8_K scale before SwarmLLM's #404 patch,
// the reference's A/B knob (vendor/candle/candle-core/src/quantized/k_quants.rs:145-152). Read once.
float q8k_scale() {
  static const float s = [] {
    const char* v = std::getenv("SWARMLLM_Q8K_SCALE");
    return (v && std::strcmp(v, "128") == 0) ? 128.0f : 127.0f;
  }();
  return s;
}

int status_of(hipError_t e) { return e == hipSuccess ? QMM_OK : QMM_DEVICE_ERROR; }

// A launch is judged by the runtime's last error afterwards; an error an
// earlier, unrelated call left behind is cleared first (mmq_entry.cu:120-122).
void clear_stale_error() { (void)hipGetLastError(); }

bool shape_ok(int type, int64_t k, int64_t n, int64_t rows) {
  const int qk = block_size(type);
  return qk != 0 && k > 0 && k % qk == 0 && n > 0 && rows > 0 && k <= (int64_t)1 << 30 && n <= ((int64_t)1 << 31) - 1;
}

// Compute units of the current device (256 on an MI355X), read once per device.
int cu_count() {
  static std::mutex mu;
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!cached[dev]) {
    hipDeviceProp_t prop;
    cached[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0
                      ? prop.multiProcessorCount
                      : 256;
    (void)hipGetLastError();
  }
  return cached[dev];
}

// The reference's few-rows line (mmq_takes_few_rows, mmq_fewest_rows_default,
// quantized/cuda.rs:775-839): K-quant products of 4 to 8 rows against a
// weight of 2 MiB or more go to the matrix cores, as do all of more than 8.
// The 32-value formats keep the decode kernels to 8 rows (their GEMM from 9:
// on MI355X the decode kernels read such a weight faster than a 128-row tile
// of 7-8 useful rows computes it).
constexpr int64_t kFewRowsLeastBytes = (int64_t)2 << 20;
constexpr int kFewRowsKQuant = 4;

// The reference's A/B switches for that line, each read once
// (quantized/cuda.rs:737-872):
//   SWARMLLM_QMATMUL_MMQ=dp4a|0|off|false   no matrix-core kernel (products
//       past the decode rows run on the decode kernels, 8 rows a launch);
//   SWARMLLM_QMATMUL_MMQ_MAX_ROWS=N         the matrix-core kernels take at most N rows;
//   SWARMLLM_QMATMUL_MMQ_MIN_ROWS=N         one few-rows line for every type
//       (N > 8: never below 9 rows);
//   SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES=B   the least weight bytes for a few-rows product (0: any);
//   SWARMLLM_QMATMUL_MMQ_CAPTURED=0|off|false  products of at most 8 rows on a
//       stream being captured stay on the decode kernels.
// A value that does not parse as a count leaves the default, as there.
struct MmqPolicy {
  bool on = true;
  int64_t max_rows = INT64_MAX;
  int64_t min_rows = -1;  // -1: per type
  int64_t few_bytes = kFewRowsLeastBytes;
  bool captured = true;
};

bool env_is_off(const char* v) {
  return v && (std::strcmp(v, "0") == 0 || std::strcmp(v, "off") == 0 || std::strcmp(v, "false") == 0);
}

// A decimal count (usize::parse: digits only, no sign or space), or -1.
int64_t env_count(const char* name) {
  const char* v = std::getenv(name);
  if (!v || !*v) return -1;
  int64_t r = 0;
  for (const char* c = v; *c; c++) {
    if (*c < '0' || *c > '9') return -1;
    if (r > (INT64_MAX - 9) / 10) return INT64_MAX;
    r = r * 10 + (*c - '0');
  }
  return r;
}

const MmqPolicy& mmq_policy() {
  static const MmqPolicy pol = [] {
    MmqPolicy p;
    const char* v = std::getenv("SWARMLLM_QMATMUL_MMQ");
    p.on = !(env_is_off(v) || (v && std::strcmp(v, "dp4a") == 0));
    const int64_t mx = env_count("SWARMLLM_QMATMUL_MMQ_MAX_ROWS");
    if (mx >= 0) p.max_rows = mx;
    p.min_rows = env_count("SWARMLLM_QMATMUL_MMQ_MIN_ROWS");
    const int64_t fb = env_count("SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES");
    if (fb >= 0) p.few_bytes = fb;
    p.captured = !env_is_off(std::getenv("SWARMLLM_QMATMUL_MMQ_CAPTURED"));
    return p;
  }();
  return pol;
}

bool is_kquant(int type) { return type == qmm::T_Q4_K || type == qmm::T_Q6_K; }

// SWARMLLM_QMATMUL_EXACT=1|on|true, read once: the exact Q4_K / Q6_K kernels
// only. Without it, three kernels feed the matrix cores a rounded product of
// a code and its sub-block scale (the single-pass Q4_K and Q6_K GEMMs from
// gemm_q4k_sp_min_rows() rows, the single-product form of the few-row Q6_K
// kernel from k = 2048), so a product's bits can depend on how many rows
// its batch has; with it, every row count sums exact int32 products.
bool env_is_on(const char* v) {
  return v && (std::strcmp(v, "1") == 0 || std::strcmp(v, "on") == 0 || std::strcmp(v, "true") == 0);
}

// The few-rows line of a type: (fewest rows, least weight bytes).
void few_rows_line(int type, int64_t& rows, int64_t& bytes) {
  const MmqPolicy& pol = mmq_policy();
  rows = pol.min_rows >= 0 ? pol.min_rows : (is_kquant(type) ? kFewRowsKQuant : qmm::gemm_b32_min_rows());
  bytes = pol.few_bytes;
}

// Types prepared on a device (qmm_prepare), a bit each: the reference's
// MMQ_FEW_ROWS_READY (quantized/cuda.rs:890-932). A product of at most 8
// rows on a stream being captured takes a matrix-core kernel only once its
// type is prepared on the current device; the first such product outside a
// capture prepares it (mmq_prepare_few_rows_once).
constexpr int kMaxDevices = 64;
std::atomic<uint32_t> g_prepared[kMaxDevices];
std::atomic<uint32_t> g_prepare_tried[kMaxDevices];

int type_bit(int type) {
  switch (type) {
    case qmm::T_Q8_0: return 1;
    case qmm::T_Q4_K: return 2;
    case qmm::T_Q6_K: return 4;
    case qmm::T_IQ4_NL: return 8;
    case qmm::T_MXFP4: return 16;
    default: return 0;
  }
}

int current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return -1;
  }
  return dev;
}

bool prepared(int type) {
  const int dev = current_device();
  return dev >= 0 && (g_prepared[dev].load(std::memory_order_acquire) & (uint32_t)type_bit(type)) != 0;
}

bool stream_is_capturing(hipStream_t st) {
  hipStreamCaptureStatus s = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(st, &s);
  if (e != hipSuccess) (void)hipGetLastError();
  return e == hipSuccess && s != hipStreamCaptureStatusNone;
}

// Whether a product of rows <= matvec_max_rows() against wbytes of weight
// goes to a matrix-core kernel (mmq_takes_few_rows, cuda.rs:823-839).
bool few_rows_take(int type, int64_t rows, int64_t wbytes, hipStream_t st) {
  int64_t fewest, least;
  few_rows_line(type, fewest, least);
  if (rows < (fewest > 2 ? fewest : 2) || wbytes < least) return false;
  if (!stream_is_capturing(st)) {
    const int dev = current_device();
    const uint32_t bit = (uint32_t)type_bit(type);
    if (dev >= 0 && !(g_prepare_tried[dev].fetch_or(bit, std::memory_order_acq_rel) & bit)) (void)qmm_prepare(type);
    return true;
  }
  return mmq_policy().captured && prepared(type);
}

bool mmq_allows(int64_t rows) {
  const MmqPolicy& pol = mmq_policy();
  return pol.on && rows <= pol.max_rows;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// The few-row matrix-core kernels (Q4_K, Q6_K): up to
// gemm_q4k_skinny_max_rows() rows past the few-rows line.
bool skinny_takes(int type, const void* w, const void* xq, int64_t n, int64_t k, int64_t rows, hipStream_t st) {
  if (!mmq_allows(rows) || rows > qmm::gemm_q4k_skinny_max_rows() || !aligned16(w) || !aligned16(xq)) return false;
  int64_t wbytes;
  if (type == qmm::T_Q4_K && qmm::gemm_q4k_skinny_fits(k, rows))
    wbytes = n * (k / 256) * 144;
  else if (type == qmm::T_Q6_K && qmm::gemm_q6k_skinny_fits(k, rows))
    wbytes = n * (k / 256) * 210;
  else
    return false;
  if (rows > qmm::matvec_max_rows()) return true;
  return few_rows_take(type, rows, wbytes, st);
}

hipError_t launch_skinny(int type, const qmm::MvTargets& t, int64_t k, const qmm::ActPlanes& p, int64_t rows,
                         hipStream_t st) {
  if (type == qmm::T_Q6_K) return qmm::launch_gemm_q6k_skinny(t, k, p, rows, (int)cu_count(), st);
  return qmm::launch_gemm_q4k_skinny(t, k, p, rows, (int)cu_count(), st);
}

// The tiled int8 matrix-core GEMMs: Q4_K and Q6_K past the skinny kernels'
// rows, Q8_0 / IQ4_NL / MXFP4 past the decode kernels' rows (or from the
// few-rows line, where SWARMLLM_QMATMUL_MMQ_MIN_ROWS moves it below); weight
// and quantized activation 16-byte aligned (their 16-byte copies), sizes
// inside their 32-bit offsets.
bool gemm_takes(int type, const void* w, const void* xq, int64_t n, int64_t k, int64_t rows, hipStream_t st) {
  if (!mmq_allows(rows) || !aligned16(w) || !aligned16(xq)) return false;
  if (type == qmm::T_Q4_K) return rows >= qmm::gemm_q4k_min_rows() && qmm::gemm_q4k_fits(n, k, rows);
  if (type == qmm::T_Q6_K) return rows >= qmm::gemm_q6k_min_rows() && qmm::gemm_q6k_fits(n, k, rows);
  if (!qmm::gemm_b32_fits(type, n, k, rows)) return false;
  if (rows > qmm::matvec_max_rows()) return true;
  return few_rows_take(type, rows, n * (k / 32) * type_size(type), st);
}

// Whether a product goes to a matrix-core kernel rather than the decode kernels.
bool matrix_takes(int type, const void* w, const void* xq, int64_t n, int64_t k, int64_t rows, hipStream_t st) {
  return gemm_takes(type, w, xq, n, k, rows, st) || skinny_takes(type, w, xq, n, k, rows, st);
}

// Q4_K: from 129 rows the single-pass GEMM (256-row tiles); 33-128 rows keep
// the exact two-pass kernel, whose 128-row tiles waste less on short batches.
hipError_t launch_gemm(int type, const void* w, int64_t n, int64_t k, const qmm::ActPlanes& p, int64_t rows,
                       float* dst, int64_t ldd, hipStream_t st) {
  if (qmm::exact_forms()) {
    if (type == qmm::T_Q6_K) return qmm::launch_gemm_q6k(w, n, k, p, rows, dst, ldd, st);
    if (type == qmm::T_Q4_K) return qmm::launch_gemm_q4k(w, n, k, p, rows, dst, ldd, st);
  }
  if (type == qmm::T_Q6_K) {
    // without a workspace for K splits, the single-pass Q6_K GEMM only where
    // its tiles fill the CUs (uncut, its per-super-block work is ~1.5x the
    // exact kernel's share of a narrow product)
    if (rows >= qmm::gemm_q4k_sp_min_rows() && qmm::gemm_q6k_sp_fits(n, k, rows) &&
        qmm::gemm_q4k_sp_splits(n, k, rows, (int)cu_count()) == 1)
      return qmm::launch_gemm_q6k_sp(w, n, k, p, rows, dst, ldd, st);
    return qmm::launch_gemm_q6k(w, n, k, p, rows, dst, ldd, st);
  }
  if (type != qmm::T_Q4_K) return qmm::launch_gemm_b32(type, w, n, k, p, rows, dst, ldd, st);
  if (rows >= qmm::gemm_q4k_sp_min_rows() && qmm::gemm_q4k_sp_fits(n, k, rows))
    return qmm::launch_gemm_q4k_sp(w, n, k, p, rows, dst, ldd, st);
  return qmm::launch_gemm_q4k(w, n, k, p, rows, dst, ldd, st);
}

// Products the single-pass Q4_K GEMM takes: those it can cut along K and
// launch several of at once (launch_gemm_q4k_sp_targets).
bool sp_takes(int type, const void* w, const void* xq, int64_t n, int64_t k, int64_t rows, hipStream_t st) {
  if ((type != qmm::T_Q4_K && type != qmm::T_Q6_K) || qmm::exact_forms()) return false;
  if (!gemm_takes(type, w, xq, n, k, rows, st) || rows < qmm::gemm_q4k_sp_min_rows()) return false;
  return type == qmm::T_Q4_K ? qmm::gemm_q4k_sp_fits(n, k, rows) : qmm::gemm_q6k_sp_fits(n, k, rows);
}

hipError_t launch_sp(int type, const qmm::MvTargets& t, int64_t k, const qmm::ActPlanes& p, int64_t rows, void* ws,
                     size_t ws_bytes, hipStream_t st) {
  return type == qmm::T_Q6_K ? qmm::launch_gemm_q6k_sp_targets(t, k, p, rows, ws, ws_bytes, (int)cu_count(), st)
                             : qmm::launch_gemm_q4k_sp_targets(t, k, p, rows, ws, ws_bytes, (int)cu_count(), st);
}

qmm::MvTargets one_target(const void* w, int64_t n, float* dst, int64_t ldd) {
  qmm::MvTargets t{};
  t.w[0] = w;
  t.dst[0] = dst;
  t.ldd[0] = ldd;
  t.row_end[0] = n;
  t.count = 1;
  return t;
}

// The streaming decode kernels (Q4_K, Q6_K at 1-2 activation rows).
bool stream_supported(int type, int64_t k, int64_t rows) {
  if (qmm::mv_b32_rows_supported(type, k, rows)) return true;
  if (type == qmm::T_Q4_K) return qmm::mv_q4k_rows_supported(k, rows);
  if (type == qmm::T_Q6_K) return qmm::mv_q6k_rows_supported(k, rows);
  return false;
}

// Launch shape of the Q4_K decode kernel for n_total weight rows, in 16-wave
// workgroups (one activation fill per 16 waves): a row per wave up to 16
// waves a CU; beyond that, about 1.5 rows per wave up to 32 waves a CU, the
// next row's loads in flight whenever a wave has more than one row.
qmm::MvShape stream_shape(int64_t n_total, int64_t k) {
  const int64_t cus = cu_count();
  // a row per wave while the rows fit one 16-wave workgroup a CU (o, 4096
  // rows: 5.5 us against 6.2 us for 2736 waves with the next row in flight)
  if (n_total <= cus * 16) return qmm::MvShape{(n_total + 15) / 16 * 16, 16, false};
  // Rows of more than 4096 values hold twice the registers: one 16-wave
  // workgroup a CU is resident, so the grid is one round of cus * 16 waves
  // with the rows spread over it (8192 rows of 8192: two a wave; 5472 waves
  // ran as 256 workgroups and then 86 on a third of the GPU).
  if (k > 4096) return qmm::MvShape{cus * 16, 16, true};
  int64_t waves = n_total * 2 / 3;
  if (waves < 1024) waves = 1024;
  if (waves > cus * 32) waves = cus * 32;
  waves = (waves + 15) / 16 * 16;
  return qmm::MvShape{waves, 16, n_total > waves};
}

// One streaming launch over up to kMaxTargets weights.
hipError_t launch_stream_targets(int type, int count, const void* const* w, const int64_t* n, float* const* dst,
                                 const int64_t* ldd, int64_t k, int64_t rows, const float* x, int64_t x_stride,
                                 const qmm::ActPlanes* pre, hipStream_t st) {
  qmm::MvTargets t{};
  int64_t end = 0;
  for (int i = 0; i < count; i++) {
    t.w[i] = w[i];
    t.dst[i] = dst[i];
    t.ldd[i] = ldd[i];
    end += n[i];
    t.row_end[i] = end;
  }
  t.count = count;
  if (type == qmm::T_Q6_K) return qmm::launch_mv_q6k_rows(t, k, rows, x, x_stride, pre, q8k_scale(), (int)cu_count(), st);
  if (type != qmm::T_Q4_K) return qmm::launch_mv_b32_rows(type, t, k, rows, x, x_stride, pre, (int)cu_count(), st);
  return qmm::launch_mv_q4k_rows(t, k, rows, x, x_stride, pre, q8k_scale(), stream_shape(end, k), st);
}

}  // namespace

namespace qmm {
bool exact_forms() {
  static const bool on = env_is_on(std::getenv("SWARMLLM_QMATMUL_EXACT"));
  return on;
}

namespace {
std::atomic<const char*> g_last_kernel{""};

// The kernels that may ask for more than 64 KiB of LDS (registered as the
// library loads) and the (device, kernel) pairs whose limit is raised.
std::mutex& lds_mu() {
  static std::mutex m;
  return m;
}
std::vector<const void*>& lds_kernels() {
  static std::vector<const void*> v;
  return v;
}
std::set<std::pair<int, const void*>>& lds_raised() {
  static std::set<std::pair<int, const void*>> s;
  return s;
}
}  // namespace
void note_launch(const char* what) { g_last_kernel.store(what, std::memory_order_relaxed); }

bool big_lds_register(const void* fn) {
  std::lock_guard<std::mutex> lock(lds_mu());
  lds_kernels().push_back(fn);
  return true;
}

hipError_t raise_lds_limit(const void* fn) {
  int dev = -1;
  const hipError_t g = hipGetDevice(&dev);
  if (g != hipSuccess) return g;
  std::lock_guard<std::mutex> lock(lds_mu());
  if (lds_raised().count({dev, fn})) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (e == hipSuccess) lds_raised().insert({dev, fn});
  return e;
}

hipError_t raise_all_lds_limits() {
  std::vector<const void*> all;
  {
    std::lock_guard<std::mutex> lock(lds_mu());
    all = lds_kernels();
  }
  for (const void* fn : all) {
    const hipError_t e = raise_lds_limit(fn);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
}  // namespace qmm

extern "C" {

const char* qmm_last_kernel(void) { return qmm::g_last_kernel.load(std::memory_order_relaxed); }

int qmm_available(void) {
  static std::mutex mu;
  static int cached[64];
  static bool known[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!known[dev]) {
    hipDeviceProp_t prop;
    int ok = 0;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    (void)hipGetLastError();
    cached[dev] = ok;
    known[dev] = true;
  }
  return cached[dev];
}

int qmm_prepare(int type) {
  const uint32_t bit = (uint32_t)type_bit(type);
  if (!bit) return QMM_UNSUPPORTED;
  const int dev = current_device();
  if (dev < 0) return QMM_DEVICE_ERROR;
  if (!qmm_available()) return QMM_NO_TILE;
  (void)cu_count();
  (void)mmq_policy();
  const bool scratch = qmm::noalloc_prepare();
  const hipError_t e = qmm::raise_all_lds_limits();
  (void)hipGetLastError();  // not sticky: leave nothing for a later check to read
  if (!scratch || e != hipSuccess) return QMM_DEVICE_ERROR;
  g_prepared[dev].fetch_or(bit, std::memory_order_acq_rel);
  return QMM_OK;
}

int qmm_prepared(int type) { return prepared(type) ? 1 : 0; }

// Every product here sums in int32 / f32 (no f16 accumulator to widen).
int qmm_accumulate_in_f32(int type) { return type_bit(type) ? QMM_OK : QMM_UNSUPPORTED; }

int qmm_block_size(int type) { return block_size(type); }

size_t qmm_type_bytes(int type, int64_t nelem) {
  const int qk = block_size(type);
  if (qk == 0 || nelem < 0 || nelem % qk) return 0;
  return (size_t)(nelem / qk) * (size_t)type_size(type);
}

int qmm_act_layout(int type, int64_t rows) {
  (void)rows;
  switch (type) {
    case qmm::T_Q4_K: case qmm::T_Q6_K: return QMM_ACT_Q8K;
    case qmm::T_Q8_0: case qmm::T_IQ4_NL: case qmm::T_MXFP4: return QMM_ACT_Q8_0;
    default: return -1;
  }
}

size_t qmm_act_bytes(int layout, int64_t k, int64_t rows) {
  if ((layout != QMM_ACT_Q8K && layout != QMM_ACT_Q8_0) || k <= 0 || rows <= 0) return 0;
  if (k % (layout == QMM_ACT_Q8K ? 256 : 32)) return 0;
  return qmm::act_bytes(layout, k, rows);
}

int qmm_act_planes(int layout, int64_t k, int64_t rows, size_t* codes_off, size_t* scales_off, size_t* sums_off) {
  if (qmm_act_bytes(layout, k, rows) == 0) return QMM_UNSUPPORTED;
  size_t so = 0, uo = 0;
  qmm::act_plane_offsets(layout, k, rows, &so, &uo);
  if (codes_off) *codes_off = 0;
  if (scales_off) *scales_off = so;
  if (sums_off) *sums_off = uo;
  return QMM_OK;
}

int qmm_quantize_act(const float* x, void* xq, int layout, int64_t k, int64_t rows, int64_t stride, int64_t stream) {
  if (qmm_act_bytes(layout, k, rows) == 0 || stride < k || x == nullptr || xq == nullptr) return QMM_UNSUPPORTED;
  clear_stale_error();
  return status_of(qmm::launch_act_quantize(layout, x, stride, k, rows, xq, q8k_scale(), (hipStream_t)stream));
}

int qmm_matvec_max_rows(void) { return qmm::matvec_max_rows(); }

void qmm_set_force_dmmv(int on) { g_force_dmmv.store(on != 0, std::memory_order_relaxed); }
int qmm_force_dmmv(void) { return g_force_dmmv.load(std::memory_order_relaxed) ? 1 : 0; }

int qmm_mmq_few_rows_line(int type, int64_t* rows, int64_t* bytes) {
  if (block_size(type) == 0 || !rows || !bytes) return QMM_UNSUPPORTED;
  few_rows_line(type, *rows, *bytes);
  return QMM_OK;
}

int64_t qmm_mmq_max_rows(void) {
  const MmqPolicy& pol = mmq_policy();
  return pol.on ? pol.max_rows : 0;
}

int qmm_mmq_captured(void) { return mmq_policy().captured ? 1 : 0; }

int qmm_exact_forms(void) { return qmm::exact_forms() ? 1 : 0; }

int qmm_matvec(int type, const void* w, const void* xq, float* dst, int64_t ldd, int64_t k, int64_t n, int64_t rows,
               int64_t stream) {
  if (!shape_ok(type, k, n, rows) || rows > qmm::matvec_max_rows() || ldd < n || !w || !xq || !dst)
    return QMM_UNSUPPORTED;
  const int layout = qmm_act_layout(type, rows);
  const qmm::ActPlanes p = qmm::act_planes(layout, (void*)xq, k, rows);
  clear_stale_error();
  hipError_t e;
  if (stream_supported(type, k, rows))
    e = launch_stream_targets(type, 1, &w, &n, &dst, &ldd, k, rows, nullptr, 0, &p, (hipStream_t)stream);
  else
    e = qmm::launch_matvec(type, w, n, k, p, rows, dst, ldd, (hipStream_t)stream);
  if (e == hipSuccess) g_matvec_launches.fetch_add(1, std::memory_order_relaxed);
  return status_of(e);
}

// One product from an activation already quantized into planes p (buffer
// xq): the matrix-core kernels past the few-rows line, else the decode
// kernels a chunk of at most matvec_max_rows() rows at a time.
int launch_product(int type, const void* w, int64_t n, int64_t k, const void* xq, const qmm::ActPlanes& p,
                   int layout, int64_t rows, float* dst, int64_t ldd, hipStream_t st) {
  if (gemm_takes(type, w, xq, n, k, rows, st)) {
    if (launch_gemm(type, w, n, k, p, rows, dst, ldd, st) != hipSuccess) return QMM_DEVICE_ERROR;
    g_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  if (skinny_takes(type, w, xq, n, k, rows, st)) {
    qmm::MvTargets t{};
    t.w[0] = w;
    t.dst[0] = dst;
    t.ldd[0] = ldd;
    t.row_end[0] = n;
    t.count = 1;
    if (launch_skinny(type, t, k, p, rows, st) != hipSuccess) return QMM_DEVICE_ERROR;
    g_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  const int64_t step = qmm::matvec_max_rows();
  for (int64_t r0 = 0; r0 < rows; r0 += step) {
    const int64_t nr = rows - r0 < step ? rows - r0 : step;
    const qmm::ActPlanes pr = qmm::act_rows(layout, p, k, r0);
    float* d = dst + r0 * ldd;
    const hipError_t e = stream_supported(type, k, nr)
                             ? launch_stream_targets(type, 1, &w, &n, &d, &ldd, k, nr, nullptr, 0, &pr, st)
                             : qmm::launch_matvec(type, w, n, k, pr, nr, d, ldd, st);
    if (e != hipSuccess) return QMM_DEVICE_ERROR;
    g_matvec_launches.fetch_add(1, std::memory_order_relaxed);
  }
  return QMM_OK;
}

int qmm_matmul(int type, const void* w, const void* xq, float* dst, int64_t ldd, int64_t k, int64_t n, int64_t rows,
               int64_t stream) {
  if (!shape_ok(type, k, n, rows) || ldd < n || !w || !xq || !dst) return QMM_UNSUPPORTED;
  const int layout = qmm_act_layout(type, rows);
  const qmm::ActPlanes p = qmm::act_planes(layout, (void*)xq, k, rows);
  clear_stale_error();
  return launch_product(type, w, n, k, xq, p, layout, rows, dst, ldd, (hipStream_t)stream);
}

int qmm_forward(int type, const void* w, const float* x, int64_t x_stride, float* dst, int64_t ldd, void* workspace,
                size_t workspace_bytes, size_t* need, int64_t k, int64_t n, int64_t rows, int launch, int64_t stream) {
  if (!shape_ok(type, k, n, rows) || need == nullptr || ldd < n || x_stride < k) return QMM_UNSUPPORTED;
  const int layout = qmm_act_layout(type, rows);
  const size_t bytes = qmm::act_bytes(layout, k, rows);
  const hipStream_t st = (hipStream_t)stream;
  // a single-pass GEMM that leaves CUs idle is cut along K when the
  // workspace also holds its split slots (need reports them; with only the
  // activation's bytes it runs uncut)
  const size_t split = sp_takes(type, w, workspace, n, k, rows, st)
                           ? qmm::gemm_q4k_sp_split_bytes(one_target(w, n, dst, ldd), k, rows, (int)cu_count())
                           : 0;
  *need = split ? qmm::align_up(bytes, 256) + split : bytes;
  if (!launch) return QMM_OK;
  if (g_fail_next.exchange(false)) return QMM_NO_ROOM;
  if (workspace_bytes < bytes || workspace == nullptr) return QMM_WORKSPACE_TOO_SMALL;
  if (!w || !x || !dst) return QMM_UNSUPPORTED;
  clear_stale_error();
  if (g_force_dmmv.load(std::memory_order_relaxed))
    return status_of(qmm::launch_dmmv(type, w, n, k, x, x_stride, rows, dst, ldd, st));
  if (stream_supported(type, k, rows) && qmm::mv_q4k_rows_fusable(x, x_stride) &&
      !matrix_takes(type, w, workspace, n, k, rows, st)) {
    // the activation is quantized inside the product's own launch
    const hipError_t e = launch_stream_targets(type, 1, &w, &n, &dst, &ldd, k, rows, x, x_stride, nullptr, st);
    if (e != hipSuccess) return QMM_DEVICE_ERROR;
    g_matvec_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  if (qmm::launch_act_quantize(layout, x, x_stride, k, rows, workspace, q8k_scale(), st) != hipSuccess)
    return QMM_DEVICE_ERROR;
  const qmm::ActPlanes p = qmm::act_planes(layout, workspace, k, rows);
  // Q6_K takes the single-pass GEMM only cut as planned (uncut, a narrow
  // product runs faster on the exact kernel)
  if (sp_takes(type, w, workspace, n, k, rows, st) &&
      (type == qmm::T_Q4_K || split == 0 || workspace_bytes >= *need)) {
    const size_t off = qmm::align_up(bytes, 256);
    void* sws = workspace_bytes > off ? (char*)workspace + off : nullptr;
    if (launch_sp(type, one_target(w, n, dst, ldd), k, p, rows, sws, workspace_bytes > off ? workspace_bytes - off : 0,
                  st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  return launch_product(type, w, n, k, workspace, p, layout, rows, dst, ldd, st);
}

int qmm_forward_shared(int type, int count, const void* const* w, const int64_t* n, float* const* dst,
                       const int64_t* ldd, const float* x, int64_t x_stride, void* workspace, size_t workspace_bytes,
                       size_t* need, int64_t k, int64_t rows, int launch, int64_t stream) {
  if (count < 1 || !w || !n || !dst || !ldd || need == nullptr || x_stride < k) return QMM_UNSUPPORTED;
  for (int i = 0; i < count; i++)
    if (!shape_ok(type, k, n[i], rows) || ldd[i] < n[i]) return QMM_UNSUPPORTED;
  const int layout = qmm_act_layout(type, rows);
  const size_t bytes = qmm::act_bytes(layout, k, rows);
  const hipStream_t st = (hipStream_t)stream;
  // the single-pass GEMM's products go kMaxTargets to a launch; their split
  // slots follow the activation (one launch's worth, reused launch after launch)
  size_t split = 0;
  {
    qmm::MvTargets g{};
    int64_t end = 0;
    for (int i = 0; i <= count; i++) {
      if (i < count && sp_takes(type, w[i], workspace, n[i], k, rows, st)) {
        g.w[g.count] = w[i];
        g.dst[g.count] = dst[i];
        g.ldd[g.count] = ldd[i];
        end += n[i];
        g.row_end[g.count] = end;
        g.count++;
      }
      if (g.count == qmm::kMaxTargets || (i == count && g.count > 0)) {
        const size_t b = qmm::gemm_q4k_sp_split_bytes(g, k, rows, (int)cu_count());
        split = b > split ? b : split;
        g = qmm::MvTargets{};
        end = 0;
      }
    }
  }
  *need = split ? qmm::align_up(bytes, 256) + split : bytes;
  if (!launch) return QMM_OK;
  if (g_fail_next.exchange(false)) return QMM_NO_ROOM;
  if (!x) return QMM_UNSUPPORTED;
  for (int i = 0; i < count; i++)
    if (!w[i] || !dst[i]) return QMM_UNSUPPORTED;
  clear_stale_error();
  if (g_force_dmmv.load(std::memory_order_relaxed)) {
    for (int i = 0; i < count; i++)
      if (qmm::launch_dmmv(type, w[i], n[i], k, x, x_stride, rows, dst[i], ldd[i], st) != hipSuccess)
        return QMM_DEVICE_ERROR;
    return QMM_OK;
  }
  bool fused = stream_supported(type, k, rows) && qmm::mv_q4k_rows_fusable(x, x_stride);
  for (int i = 0; fused && i < count; i++) fused = !matrix_takes(type, w[i], workspace, n[i], k, rows, st);
  if (fused) {
    // one launch per kMaxTargets weights, each quantizing the activation in LDS
    for (int i0 = 0; i0 < count; i0 += qmm::kMaxTargets) {
      const int c = count - i0 < qmm::kMaxTargets ? count - i0 : qmm::kMaxTargets;
      if (launch_stream_targets(type, c, w + i0, n + i0, dst + i0, ldd + i0, k, rows, x, x_stride, nullptr, st) !=
          hipSuccess)
        return QMM_DEVICE_ERROR;
      g_matvec_launches.fetch_add(1, std::memory_order_relaxed);
    }
    return QMM_OK;
  }
  // otherwise: the activation quantized once into the workspace, then each product
  if (workspace_bytes < bytes || workspace == nullptr) return QMM_WORKSPACE_TOO_SMALL;
  if (qmm::launch_act_quantize(layout, x, x_stride, k, rows, workspace, q8k_scale(), st) != hipSuccess)
    return QMM_DEVICE_ERROR;
  const qmm::ActPlanes p = qmm::act_planes(layout, workspace, k, rows);
  // the weights the skinny kernel takes share its launches (kMaxTargets
  // each), and so do those the single-pass GEMM takes
  qmm::MvTargets grp{}, spg{};
  int64_t end = 0, spend = 0;
  auto flush = [&]() -> int {
    if (grp.count == 0) return QMM_OK;
    if (launch_skinny(type, grp, k, p, rows, st) != hipSuccess) return QMM_DEVICE_ERROR;
    g_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    grp = qmm::MvTargets{};
    end = 0;
    return QMM_OK;
  };
  const size_t off = qmm::align_up(bytes, 256);
  void* sws = workspace_bytes > off ? (char*)workspace + off : nullptr;
  const size_t sbytes = workspace_bytes > off ? workspace_bytes - off : 0;
  auto flush_sp = [&]() -> int {
    if (spg.count == 0) return QMM_OK;
    if (launch_sp(type, spg, k, p, rows, sws, sbytes, st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    spg = qmm::MvTargets{};
    spend = 0;
    return QMM_OK;
  };
  const bool sp_ok = type == qmm::T_Q4_K || split == 0 || workspace_bytes >= *need;
  for (int i = 0; i < count; i++) {
    if (sp_ok && sp_takes(type, w[i], workspace, n[i], k, rows, st)) {
      spg.w[spg.count] = w[i];
      spg.dst[spg.count] = dst[i];
      spg.ldd[spg.count] = ldd[i];
      spend += n[i];
      spg.row_end[spg.count] = spend;
      if (++spg.count == qmm::kMaxTargets && flush_sp() != QMM_OK) return QMM_DEVICE_ERROR;
      continue;
    }
    if (!gemm_takes(type, w[i], workspace, n[i], k, rows, st) &&
        skinny_takes(type, w[i], workspace, n[i], k, rows, st)) {
      grp.w[grp.count] = w[i];
      grp.dst[grp.count] = dst[i];
      grp.ldd[grp.count] = ldd[i];
      end += n[i];
      grp.row_end[grp.count] = end;
      if (++grp.count == qmm::kMaxTargets && flush() != QMM_OK) return QMM_DEVICE_ERROR;
      continue;
    }
    const int r = launch_product(type, w[i], n[i], k, workspace, p, layout, rows, dst[i], ldd[i], st);
    if (r != QMM_OK) return r;
  }
  if (flush_sp() != QMM_OK) return QMM_DEVICE_ERROR;
  return flush();
}

int qmm_forward_glu(int type, int act, const void* w_gate, const void* w_up, const float* x, int64_t x_stride,
                    float* dst, int64_t ldd, void* workspace, size_t workspace_bytes, size_t* need, int64_t k,
                    int64_t n, int64_t rows, int launch, int64_t stream) {
  if (!shape_ok(type, k, n, rows) || act < QMM_GLU_SILU || act > QMM_GLU_GELU || need == nullptr || ldd < n ||
      x_stride < k)
    return QMM_UNSUPPORTED;
  // workspace: the quantized activation, then the gate and up products of
  // the two-launch form
  const int layout = qmm_act_layout(type, rows);
  const size_t abytes = qmm::act_bytes(layout, k, rows);
  const size_t obytes = qmm::align_up((size_t)(rows * n) * 4, 256);
  const size_t bytes = abytes + 2 * obytes;
  *need = bytes;
  if (!launch) return QMM_OK;
  if (g_fail_next.exchange(false)) return QMM_NO_ROOM;
  if (!w_gate || !w_up || !x || !dst) return QMM_UNSUPPORTED;
  const hipStream_t st = (hipStream_t)stream;
  clear_stale_error();
  if (type == qmm::T_Q4_K && !g_force_dmmv.load(std::memory_order_relaxed) && qmm::mv_q4k_glu_supported(k, rows) &&
      qmm::mv_q4k_rows_fusable(x, x_stride) &&
      !matrix_takes(type, w_gate, workspace, n, k, rows, st) && !matrix_takes(type, w_up, workspace, n, k, rows, st)) {
    if (qmm::launch_mv_q4k_glu(act, w_gate, w_up, n, k, rows, x, x_stride, nullptr, q8k_scale(), dst, ldd,
                               cu_count(), st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_matvec_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  if (workspace_bytes < bytes || workspace == nullptr) return QMM_WORKSPACE_TOO_SMALL;
  float* gbuf = (float*)((char*)workspace + abytes);
  float* ubuf = (float*)((char*)gbuf + obytes);
  const void* w[2] = {w_gate, w_up};
  const int64_t ns[2] = {n, n};
  float* outs[2] = {gbuf, ubuf};
  size_t need2 = 0;
  const int r = qmm_forward_shared(type, 2, w, ns, outs, ns, x, x_stride, workspace, abytes, &need2, k, rows, 1,
                                   stream);
  if (r != QMM_OK) return r;
  return status_of(qmm::launch_glu(act, gbuf, n, ubuf, n, dst, ldd, n, rows, st));
}

int qmm_glu(int act, const float* gate, const float* up, float* out, int64_t n, int64_t stream) {
  if (act < QMM_GLU_SILU || act > QMM_GLU_GELU || n < 0 || (n > 0 && (!gate || !up || !out))) return QMM_UNSUPPORTED;
  clear_stale_error();
  return status_of(qmm::launch_glu(act, gate, n, up, n, out, n, n, 1, (hipStream_t)stream));
}

int qmm_dequantize(int type, const void* w, void* out, int out_f16, int64_t nelem, int64_t stream) {
  if (qmm_type_bytes(type, nelem) == 0 || !w || !out) return QMM_UNSUPPORTED;
  clear_stale_error();
  return status_of(qmm::launch_dequantize(type, w, out, out_f16, nelem, (hipStream_t)stream));
}

size_t qmm_quantize_scratch_bytes(int type, int64_t nelem) {
  if (qmm_type_bytes(type, nelem) == 0) return 0;
  return qmm::weight_quantize_scratch_bytes(type, nelem);
}

int qmm_quantize_weights(int type, const float* x, void* w, int64_t nelem, void* scratch, size_t scratch_bytes,
                         int64_t stream) {
  if (qmm_type_bytes(type, nelem) == 0 || !x || !w) return QMM_UNSUPPORTED;
  if (scratch_bytes < qmm::weight_quantize_scratch_bytes(type, nelem)) return QMM_WORKSPACE_TOO_SMALL;
  clear_stale_error();
  return status_of(qmm::launch_weight_quantize(type, x, w, nelem, scratch, (hipStream_t)stream));
}

int qmm_moe_forward(int type, const void* w, int num_experts, const float* x, int64_t x_stride,
                    const int32_t* sorted_ids, const int32_t* expert_ids, const float* topk_w, int topk, float* dst,
                    int64_t ldd, void* workspace, size_t workspace_bytes, size_t* need, int64_t k, int64_t n,
                    int64_t size_m, int launch, int64_t stream) {
  if (!qmm::moe_supported(type, k) || !shape_ok(type, k, n, size_m) || need == nullptr || ldd < n || x_stride < k ||
      num_experts < 1 || topk < 1 || (topk_w == nullptr && size_m % topk != 0) || size_m > ((int64_t)1 << 30))
    return QMM_UNSUPPORTED;
  const int64_t in_rows = topk_w ? size_m : size_m / topk;
  const int layout = qmm::moe_act_layout(type);
  const size_t act = (qmm::act_bytes(layout, k, in_rows) + 255) / 256 * 256;
  const size_t bytes = act + qmm::moe_runs_bytes(size_m);
  *need = bytes;
  if (!launch) return QMM_OK;
  if (g_fail_next.exchange(false)) return QMM_NO_ROOM;
  if (workspace_bytes < bytes || workspace == nullptr) return QMM_WORKSPACE_TOO_SMALL;
  if (!w || !x || !dst || !sorted_ids || !expert_ids) return QMM_UNSUPPORTED;
  const hipStream_t st = (hipStream_t)stream;
  clear_stale_error();
  if (qmm::moe_fp4_fused_takes(type, k, size_m)) {
    if (qmm::launch_moe_fp4_fused(w, num_experts, n, k, x, x_stride, expert_ids, sorted_ids, topk_w, topk, size_m, dst,
                                  ldd, st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_moe_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  if (layout == qmm::ACT_Q8K && qmm::moe_kq_fused_takes(type, k, size_m)) {
    if (qmm::launch_moe_kq_fused(type, w, num_experts, n, k, x, x_stride, expert_ids, sorted_ids, topk_w, topk, size_m,
                                 dst, ldd, q8k_scale(), (int)cu_count(), st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_moe_launches.fetch_add(1, std::memory_order_relaxed);
    return QMM_OK;
  }
  // the activation's planes (Q8_K for Q4_K / Q6_K, else Q8_0) and the run
  // table, one launch; then the grouped kernel
  int32_t* runs = (int32_t*)((char*)workspace + act);
  if (qmm::launch_act_quantize_moe(layout, x, x_stride, k, in_rows, workspace, expert_ids, size_m, runs, q8k_scale(),
                                   st) != hipSuccess)
    return QMM_DEVICE_ERROR;
  const qmm::ActPlanes p = qmm::act_planes(layout, workspace, k, in_rows);
  const hipError_t e =
      layout == qmm::ACT_Q8K
          ? qmm::launch_moe_kq(type, w, num_experts, n, k, p, runs, sorted_ids, topk_w, topk, size_m, dst, ldd,
                               (int)cu_count(), st)
          : qmm::launch_moe(type, w, num_experts, n, k, p, runs, sorted_ids, topk_w, topk, size_m, dst, ldd,
                            (int)cu_count(), st);
  if (e != hipSuccess) return QMM_DEVICE_ERROR;
  g_moe_launches.fetch_add(1, std::memory_order_relaxed);
  return QMM_OK;
}

uint64_t qmm_moe_launches(void) { return g_moe_launches.load(std::memory_order_relaxed); }

int qmm_moe_forward_prefill(int type, const void* w, int num_experts, const void* x, int x_dtype, int64_t x_stride,
                            const int32_t* sorted_ids, const int32_t* expert_ids, const float* topk_w, int topk,
                            float* dst, int64_t ldd, void* workspace, size_t workspace_bytes, size_t* need, int64_t k,
                            int64_t n, int64_t size_m, int launch, int64_t stream) {
  if (!qmm::moe_pf_supported(type, k) || !shape_ok(type, k, n, size_m) || need == nullptr || ldd < n ||
      x_stride < k || num_experts < 1 || topk < 1 || (topk_w == nullptr && size_m % topk != 0) ||
      size_m > ((int64_t)1 << 30) || x_dtype < QMM_X_F16 || x_dtype > QMM_X_F32)
    return QMM_UNSUPPORTED;
  const int64_t in_rows = topk_w ? size_m : size_m / topk;
  // 32-bit byte offsets inside the kernel: an expert's weights, the 16-bit rows
  if (n * qmm::moe_pf_row_bytes(type, k) >= ((int64_t)1 << 31) || in_rows * k * 2 >= ((int64_t)1 << 31))
    return QMM_UNSUPPORTED;
  const size_t runs_b = qmm::align_up(qmm::moe_runs_bytes(size_m), 256);
  const size_t chunks_b = qmm::align_up(qmm::moe_pf_chunks_bytes(size_m), 256);
  const size_t xo_b = qmm::align_up((size_t)(in_rows * k * 2), 256);
  *need = runs_b + chunks_b + xo_b;
  if (!launch) return QMM_OK;
  if (g_fail_next.exchange(false)) return QMM_NO_ROOM;
  if (workspace_bytes < *need || workspace == nullptr) return QMM_WORKSPACE_TOO_SMALL;
  if (!w || !x || !dst || !sorted_ids || !expert_ids || !qmm::moe_pf_weights_ok(type, w)) return QMM_UNSUPPORTED;
  const hipStream_t st = (hipStream_t)stream;
  clear_stale_error();
  int32_t* runs = (int32_t*)workspace;
  int32_t* chunks = (int32_t*)((char*)workspace + runs_b);
  uint16_t* xo = (uint16_t*)((char*)workspace + runs_b + chunks_b);
  // A 16-bit input with 16-byte aligned rows is read in place; an f32 input
  // is rounded to f16 (the reference's caller converts a prompt's input to
  // f16, moe_card.rs:113-121) and any other is copied aligned, in the
  // prologue that writes the routing tables.
  const bool direct = x_dtype != QMM_X_F32 && ((uintptr_t)x & 15) == 0 && x_stride % 8 == 0 &&
                      in_rows * x_stride * 2 < ((int64_t)1 << 31);
  const int kind = direct ? -1 : x_dtype == QMM_X_F32 ? 2 : x_dtype;
  if (qmm::launch_moe_pf_prep(expert_ids, size_m, runs, chunks, x, kind, x_stride, k, in_rows, xo, (int)cu_count(),
                              st) != hipSuccess)
    return QMM_DEVICE_ERROR;
  const hipError_t e = qmm::launch_moe_pf(type, x_dtype == QMM_X_BF16, w, num_experts, n, k,
                                          direct ? (const uint16_t*)x : xo, direct ? x_stride : k, chunks, sorted_ids,
                                          topk_w, topk, size_m, dst, ldd, st);
  if (e != hipSuccess) return QMM_DEVICE_ERROR;
  g_moe_prefill_launches.fetch_add(1, std::memory_order_relaxed);
  return QMM_OK;
}

uint64_t qmm_moe_prefill_launches(void) { return g_moe_prefill_launches.load(std::memory_order_relaxed); }

size_t qmm_wire_bytes(int64_t n) {
  const int64_t b = qmm::wire_bytes(n);
  return b < 0 ? 0 : (size_t)b;
}

int qmm_wire_encode(const float* x, int64_t n, void* out, int64_t stream) {
  if (n < 0 || qmm::wire_bytes(n) < 0 || (n > 0 && (!x || !out))) return QMM_UNSUPPORTED;
  if (n == 0) return QMM_OK;
  clear_stale_error();
  return status_of(qmm::launch_wire_encode(x, n, out, (hipStream_t)stream));
}

int qmm_wire_decode(const void* in, size_t in_bytes, int64_t n, float* out, int64_t stream) {
  // the reference rejects a payload whose length is not the one n values take
  // (dequantize_q8_0, src/inference/quant.rs:65-77)
  const int64_t want = qmm::wire_bytes(n);
  if (want < 0 || (int64_t)in_bytes != want || (n > 0 && (!in || !out))) return QMM_UNSUPPORTED;
  if (n == 0) return QMM_OK;
  clear_stale_error();
  return status_of(qmm::launch_wire_decode(in, n, out, (hipStream_t)stream));
}

void qmm_fail_next_launch(void) { g_fail_next.store(true); }

int qmm_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float std, int64_t stream) {
  if (!out || n < 0) return QMM_UNSUPPORTED;
  if (n == 0) return QMM_OK;
  clear_stale_error();
  return status_of(qmm::launch_fill_normal(out, n, seed, mean, std, (hipStream_t)stream));
}

uint64_t qmm_matvec_launches(void) { return g_matvec_launches.load(); }
uint64_t qmm_gemm_launches(void) { return g_gemm_launches.load(); }

}  // extern "C"
