// gguf.hip — GGUF files into device memory (host code; no kernels).
//
// The reader restates candle's gguf_file::Content::read
// (vendor/candle/candle-core/src/quantized/gguf_file.rs:415-487): magic
// "GGUF" (either byte order), versions 1-3 (v1 with 32-bit counts, string
// lengths and dimensions), the metadata key/value pairs of the 13 value
// types (:183-395, strings with trailing NULs dropped, :120-135), the tensor
// infos (name, dimensions outermost first, ggml type, offset), and the start
// of the tensor data: the position after the infos rounded up to
// general.alignment (U8/U16/U32, or a non-negative I8/I16/I32), 32 without it.
//
// A tensor is loaded as ggml_file::qtensor_read / cuda::load_quantized_read
// load one (ggml_file.rs:220-256, cuda.rs:1846-2075): its bytes read from the
// file into a device buffer that holds MATRIX_ROW_PADDING = 512 values' worth
// of blocks more, zeroed (cuda.rs:43). The read goes through two pinned
// staging buffers the process keeps: chunk c is read into one while chunk
// c - 1 is copied from the other (with_pinned_load_staging, cuda.rs:1966-2018;
// qmm_pinned_load_chunks counts the chunks). The reference's A/B switches,
// read once: SWARMLLM_LOAD_PINNED=0 copies through one pageable staging
// buffer instead, a chunk at a time, each copy done with its source before
// the next read (load_quantized_read, cuda.rs:2025-2069);
// SWARMLLM_LOAD_READ=fresh reads each tensor through a fresh host buffer of
// its whole size and copies it at once (gguf_file.rs:57-63).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/qmm.h"

namespace {

constexpr uint64_t kDefaultAlignment = 32;
constexpr int64_t kRowPadding = 512;
constexpr size_t kChunk = (size_t)16 << 20;

// block size and bytes a block of the ggml types a GGUF may name (candle's
// GgmlDType::block_size / type_size, quantized/mod.rs:421-461)
bool type_shape(int t, int64_t& bs, int64_t& ts) {
  switch (t) {
    case 0: bs = 1; ts = 4; return true;      // F32
    case 1: bs = 1; ts = 2; return true;      // F16
    case 2: bs = 32; ts = 18; return true;    // Q4_0
    case 3: bs = 32; ts = 20; return true;    // Q4_1
    case 6: bs = 32; ts = 22; return true;    // Q5_0
    case 7: bs = 32; ts = 24; return true;    // Q5_1
    case 8: bs = 32; ts = 34; return true;    // Q8_0
    case 9: bs = 32; ts = 36; return true;    // Q8_1
    case 10: bs = 256; ts = 84; return true;  // Q2K
    case 11: bs = 256; ts = 110; return true; // Q3K
    case 12: bs = 256; ts = 144; return true; // Q4K
    case 13: bs = 256; ts = 176; return true; // Q5K
    case 14: bs = 256; ts = 210; return true; // Q6K
    case 15: bs = 256; ts = 292; return true; // Q8K
    case 20: bs = 32; ts = 18; return true;   // IQ4_NL
    case 23: bs = 256; ts = 136; return true; // IQ4_XS
    case 30: bs = 1; ts = 2; return true;     // BF16
    case 39: bs = 32; ts = 17; return true;   // MXFP4
    default: return false;
  }
}

struct Value {
  int type = 0;       // GGUF value type id
  int elem_type = 0;  // arrays: the element type
  int64_t i = 0;      // integers and bools (u64 as its bits)
  double f = 0.0;     // f32 / f64
  std::string s;      // strings
  std::vector<Value> items;
};

struct Tensor {
  std::string name;
  int type;
  int n_dims;
  int64_t dims[4];  // outermost first
  uint64_t offset;
  uint64_t bytes;
  int64_t nelem;
  bool whole;  // nelem is a whole number of blocks
};

// Reads fields off a FILE; any short read marks the whole parse failed.
struct Reader {
  FILE* f;
  bool ok = true;
  bool read(void* p, size_t n) {
    if (ok && n && fread(p, 1, n, f) != n) ok = false;
    return ok;
  }
  template <typename T>
  T get() {
    T v{};
    read(&v, sizeof(T));
    return v;
  }
  uint64_t count(int version) { return version == 1 ? get<uint32_t>() : get<uint64_t>(); }
  std::string str(int version) {
    const uint64_t n = count(version);
    // a string longer than what is left of any sane header is a corrupt file
    if (!ok || n > ((uint64_t)1 << 32)) {
      ok = false;
      return {};
    }
    std::string s(n, '\0');
    read(s.data(), n);
    while (!s.empty() && s.back() == '\0') s.pop_back();
    return s;
  }
};

bool read_value(Reader& r, int type, int version, Value& v, int depth) {
  v.type = type;
  switch (type) {
    case 0: v.i = r.get<uint8_t>(); break;
    case 1: v.i = r.get<int8_t>(); break;
    case 2: v.i = r.get<uint16_t>(); break;
    case 3: v.i = r.get<int16_t>(); break;
    case 4: v.i = r.get<uint32_t>(); break;
    case 5: v.i = r.get<int32_t>(); break;
    case 6: v.f = r.get<float>(); break;
    case 7: {
      const uint8_t b = r.get<uint8_t>();
      if (b > 1) return false;  // the reference rejects other bool bytes
      v.i = b;
      break;
    }
    case 8: v.s = r.str(version); break;
    case 9: {
      if (depth > 8) return false;
      v.elem_type = (int)r.get<uint32_t>();
      const uint64_t n = r.count(version);
      if (!r.ok || n > ((uint64_t)1 << 32)) return false;
      v.items.resize(n);
      for (uint64_t j = 0; j < n && r.ok; j++)
        if (!read_value(r, v.elem_type, version, v.items[j], depth + 1)) return false;
      break;
    }
    case 10: v.i = (int64_t)r.get<uint64_t>(); break;
    case 11: v.i = r.get<int64_t>(); break;
    case 12: v.f = r.get<double>(); break;
    default: return false;
  }
  return r.ok;
}

// The pinned staging pair, allocated on first use and kept for the process;
// where the runtime refuses page-locked memory, loads copy through the
// pageable staging buffer instead (as the reference's scope does).
struct Staging {
  std::mutex mu;  // loads are serialized
  void* buf[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  bool recorded[2] = {false, false};  // done[b] marks a copy out of buf[b]
  bool ready = false, refused = false;
  std::vector<uint8_t> pageable;
  bool init() {
    if (ready) return true;
    if (refused) return false;
    for (int b = 0; b < 2; b++) {
      if (hipHostMalloc(&buf[b], kChunk, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        refused = true;
        return false;
      }
    }
    ready = true;
    return true;
  }
};
Staging g_staging;
std::atomic<uint64_t> g_pinned_chunks{0};

bool env_is(const char* name, const char* value) {
  const char* v = std::getenv(name);
  return v && std::strcmp(v, value) == 0;
}
bool load_pinned() {
  static const bool on = !env_is("SWARMLLM_LOAD_PINNED", "0");
  return on;
}
bool load_fresh() {
  static const bool on = env_is("SWARMLLM_LOAD_READ", "fresh");
  return on;
}

// n bytes of the file at `at` into host memory p; false when the file ends first.
bool read_file(int fd, uint8_t* p, size_t n, uint64_t at) {
  size_t got = 0;
  while (got < n) {
    const ssize_t r = pread(fd, p + got, n - got, (off_t)(at + got));
    if (r <= 0) return false;
    got += (size_t)r;
  }
  return true;
}

// len bytes of the file at `at` into device memory d, through the staging
// the switches choose; returns with every copy issued on st (the pinned
// path), or finished (the pageable and fresh paths). Called with
// g_staging.mu held.
int copy_span(int fd, uint64_t at, uint64_t len, uint8_t* d, hipStream_t st) {
  if (len == 0) return QMM_OK;
  if (load_fresh()) {
    std::vector<uint8_t> whole;
    try {
      whole.resize((size_t)len);
    } catch (...) {
      return QMM_DEVICE_ERROR;
    }
    if (!read_file(fd, whole.data(), (size_t)len, at)) return QMM_UNSUPPORTED;
    if (hipMemcpyAsync(d, whole.data(), (size_t)len, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    return QMM_OK;
  }
  if (!load_pinned() || !g_staging.init()) {
    if (g_staging.pageable.size() < kChunk) g_staging.pageable.resize(kChunk);
    for (uint64_t done = 0; done < len; done += kChunk) {
      const size_t n = (size_t)(len - done < kChunk ? len - done : kChunk);
      if (!read_file(fd, g_staging.pageable.data(), n, at + done)) return QMM_UNSUPPORTED;
      if (hipMemcpyAsync(d + done, g_staging.pageable.data(), n, hipMemcpyHostToDevice, st) != hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return QMM_DEVICE_ERROR;
    }
    return QMM_OK;
  }
  int c = 0;
  for (uint64_t done = 0; done < len; done += kChunk, c++) {
    const size_t n = (size_t)(len - done < kChunk ? len - done : kChunk);
    const int b = c & 1;
    // the copy that last read this staging buffer has finished (also one
    // issued by an earlier span of this load)
    if (g_staging.recorded[b] && hipEventSynchronize(g_staging.done[b]) != hipSuccess) return QMM_DEVICE_ERROR;
    if (!read_file(fd, (uint8_t*)g_staging.buf[b], n, at + done)) return QMM_UNSUPPORTED;
    if (hipMemcpyAsync(d + done, g_staging.buf[b], n, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(g_staging.done[b], st) != hipSuccess)
      return QMM_DEVICE_ERROR;
    g_staging.recorded[b] = true;
    g_pinned_chunks.fetch_add(1, std::memory_order_relaxed);
  }
  return QMM_OK;
}

// Padding bytes past a device weight of `type`: MATRIX_ROW_PADDING values' worth of blocks.
int64_t pad_bytes(int64_t bs, int64_t ts) { return kRowPadding / bs * ts; }

}  // namespace

struct qmm_gguf {
  int fd = -1;
  uint64_t file_bytes = 0;
  int version = 0;
  uint64_t alignment = kDefaultAlignment;
  uint64_t data_offset = 0;
  std::vector<std::pair<std::string, Value>> kv;
  std::unordered_map<std::string, int64_t> kv_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int64_t> tensor_index;
};

extern "C" {

int qmm_gguf_open(const char* path, qmm_gguf** out) {
  if (!out) return QMM_UNSUPPORTED;
  *out = nullptr;
  if (!path) return QMM_UNSUPPORTED;
  FILE* f = fopen(path, "rb");
  if (!f) return QMM_UNSUPPORTED;
  std::unique_ptr<qmm_gguf> g(new qmm_gguf);
  Reader r{f};
  const uint32_t magic = r.get<uint32_t>();
  const uint32_t version = r.get<uint32_t>();
  bool ok = r.ok && (magic == 0x46554747u || magic == 0x47475546u) && version >= 1 && version <= 3;
  g->version = (int)version;
  if (ok) {
    const uint64_t n_tensors = r.count(g->version);
    const uint64_t n_kv = r.count(g->version);
    ok = r.ok && n_tensors < ((uint64_t)1 << 32) && n_kv < ((uint64_t)1 << 32);
    for (uint64_t i = 0; ok && i < n_kv; i++) {
      std::string key = r.str(g->version);
      const int type = (int)r.get<uint32_t>();
      Value v;
      ok = r.ok && read_value(r, type, g->version, v, 0);
      if (ok) {
        // a repeated key keeps its last value, as the reference's map insert does
        auto it = g->kv_index.find(key);
        if (it != g->kv_index.end())
          g->kv[it->second].second = std::move(v);
        else {
          g->kv_index.emplace(key, (int64_t)g->kv.size());
          g->kv.emplace_back(std::move(key), std::move(v));
        }
      }
    }
    for (uint64_t i = 0; ok && i < n_tensors; i++) {
      Tensor t{};
      t.name = r.str(g->version);
      const uint32_t nd = r.get<uint32_t>();
      ok = r.ok && nd >= 1 && nd <= 4;
      uint64_t dims[4] = {0, 0, 0, 0};
      for (uint32_t d = 0; ok && d < nd; d++) dims[d] = g->version == 1 ? r.get<uint32_t>() : r.get<uint64_t>();
      t.type = (int)r.get<uint32_t>();
      t.offset = r.get<uint64_t>();
      ok = ok && r.ok;
      if (!ok) break;
      t.n_dims = (int)nd;
      int64_t nel = 1;
      for (uint32_t d = 0; d < nd; d++) {
        t.dims[d] = (int64_t)dims[nd - 1 - d];  // GGUF stores the innermost dimension first
        if (dims[d] > ((uint64_t)1 << 40) || (nel && (int64_t)dims[d] > (((int64_t)1 << 62) / nel))) ok = false;
        nel *= (int64_t)dims[d];
      }
      int64_t bs = 0, ts = 0;
      ok = ok && type_shape(t.type, bs, ts);
      if (!ok) break;
      t.nelem = nel;
      // a count that is not a whole number of blocks fails when the tensor
      // is read, not here (TensorInfo::read, gguf_file.rs:78-84)
      // (a byte count past INT64_MAX is refused the same way)
      t.whole = nel % bs == 0 && nel / bs <= INT64_MAX / ts;
      t.bytes = t.whole ? (uint64_t)(nel / bs * ts) : 0;
      // a repeated name keeps its last info, as the reference's map insert does
      auto it = g->tensor_index.find(t.name);
      if (it != g->tensor_index.end())
        g->tensors[it->second] = t;
      else {
        g->tensor_index.emplace(t.name, (int64_t)g->tensors.size());
        g->tensors.push_back(t);
      }
    }
  }
  if (ok) {
    const long pos = ftell(f);
    uint64_t align = kDefaultAlignment;
    auto it = g->kv_index.find("general.alignment");
    if (it != g->kv_index.end()) {
      const Value& v = g->kv[it->second].second;
      const bool uns = v.type == 0 || v.type == 2 || v.type == 4;
      const bool sig = (v.type == 1 || v.type == 3 || v.type == 5) && v.i >= 0;
      if (uns || sig) align = (uint64_t)v.i;
    }
    ok = pos >= 0 && align > 0;
    g->alignment = align;
    if (ok) g->data_offset = ((uint64_t)pos + align - 1) / align * align;
  }
  fclose(f);
  if (!ok) return QMM_UNSUPPORTED;
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) return QMM_UNSUPPORTED;
  struct stat sb;
  if (fstat(g->fd, &sb) != 0 || sb.st_size < 0) return QMM_UNSUPPORTED;
  g->file_bytes = (uint64_t)sb.st_size;
  *out = g.release();
  return QMM_OK;
}

void qmm_gguf_close(qmm_gguf* g) {
  if (!g) return;
  if (g->fd >= 0) close(g->fd);
  delete g;
}

int qmm_gguf_version(const qmm_gguf* g) { return g ? g->version : 0; }
uint64_t qmm_gguf_alignment(const qmm_gguf* g) { return g ? g->alignment : 0; }
uint64_t qmm_gguf_data_offset(const qmm_gguf* g) { return g ? g->data_offset : 0; }

int64_t qmm_gguf_tensor_count(const qmm_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t qmm_gguf_find_tensor(const qmm_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : it->second;
}

const char* qmm_gguf_tensor_name(const qmm_gguf* g, int64_t i) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
  return g->tensors[i].name.c_str();
}

int qmm_gguf_tensor_info(const qmm_gguf* g, int64_t i, int* type, int* n_dims, int64_t* dims, uint64_t* offset,
                         uint64_t* bytes) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return QMM_UNSUPPORTED;
  const Tensor& t = g->tensors[i];
  if (type) *type = t.type;
  if (n_dims) *n_dims = t.n_dims;
  if (dims)
    for (int d = 0; d < 4; d++) dims[d] = d < t.n_dims ? t.dims[d] : 1;
  if (offset) *offset = t.offset;
  if (bytes) *bytes = t.bytes;
  return QMM_OK;
}

int64_t qmm_gguf_kv_count(const qmm_gguf* g) { return g ? (int64_t)g->kv.size() : 0; }

int64_t qmm_gguf_find_kv(const qmm_gguf* g, const char* key) {
  if (!g || !key) return -1;
  auto it = g->kv_index.find(key);
  return it == g->kv_index.end() ? -1 : it->second;
}

const char* qmm_gguf_kv_key(const qmm_gguf* g, int64_t i) {
  if (!g || i < 0 || i >= (int64_t)g->kv.size()) return nullptr;
  return g->kv[i].first.c_str();
}

int qmm_gguf_kv_type(const qmm_gguf* g, int64_t i, int* elem_type, int64_t* len) {
  if (!g || i < 0 || i >= (int64_t)g->kv.size()) return -1;
  const Value& v = g->kv[i].second;
  if (elem_type) *elem_type = v.type == 9 ? v.elem_type : v.type;
  if (len) *len = v.type == 9 ? (int64_t)v.items.size() : 1;
  return v.type;
}

int qmm_gguf_kv_get(const qmm_gguf* g, int64_t i, int64_t j, int64_t* iv, double* fv, const char** sv) {
  if (!g || i < 0 || i >= (int64_t)g->kv.size()) return QMM_UNSUPPORTED;
  const Value& top = g->kv[i].second;
  const Value* v = &top;
  if (top.type == 9) {
    if (j < 0 || j >= (int64_t)top.items.size()) return QMM_UNSUPPORTED;
    v = &top.items[j];
    if (v->type == 9) return QMM_UNSUPPORTED;  // arrays of arrays are not read element by element
  } else if (j != 0) {
    return QMM_UNSUPPORTED;
  }
  if (iv) *iv = v->i;
  if (fv) *fv = v->f;
  if (sv) *sv = v->type == 8 ? v->s.c_str() : nullptr;
  return QMM_OK;
}

size_t qmm_padded_bytes(int type, int64_t nelem) {
  int64_t bs = 0, ts = 0;
  if (!type_shape(type, bs, ts) || nelem < 0 || nelem % bs) return 0;
  if (nelem / bs > (INT64_MAX - pad_bytes(bs, ts)) / ts) return 0;  // the size does not fit
  return (size_t)(nelem / bs * ts + pad_bytes(bs, ts));
}

uint64_t qmm_pinned_load_chunks(void) { return g_pinned_chunks.load(std::memory_order_relaxed); }

// Where tensor t's bytes start in the file; false when they would run past
// its end (a truncated or corrupt file: refused before anything is copied).
static bool tensor_span(const qmm_gguf* g, const Tensor& t, uint64_t& base) {
  if (t.offset > UINT64_MAX - g->data_offset) return false;
  base = g->data_offset + t.offset;
  return base <= g->file_bytes && t.bytes <= g->file_bytes - base;
}

int qmm_gguf_load(const qmm_gguf* g, int64_t i, void* dst, size_t dst_bytes, int64_t stream) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size() || !dst) return QMM_UNSUPPORTED;
  const Tensor& t = g->tensors[i];
  if (!t.whole) return QMM_UNSUPPORTED;
  const size_t padded = qmm_padded_bytes(t.type, t.nelem);
  if (padded == 0) return QMM_UNSUPPORTED;
  if (dst_bytes < padded) return QMM_WORKSPACE_TOO_SMALL;
  uint64_t base = 0;
  if (!tensor_span(g, t, base)) return QMM_UNSUPPORTED;
  const hipStream_t st = (hipStream_t)stream;
  std::lock_guard<std::mutex> lock(g_staging.mu);
  (void)hipGetLastError();
  uint8_t* d = (uint8_t*)dst;
  if (hipMemsetAsync(d + t.bytes, 0, padded - t.bytes, st) != hipSuccess) return QMM_DEVICE_ERROR;
  const int rc = copy_span(g->fd, base, t.bytes, d, st);
  // the staging buffers are free for the next load, and the tensor is on the device
  const bool synced = hipStreamSynchronize(st) == hipSuccess;
  if (rc != QMM_OK) return rc;
  return synced ? QMM_OK : QMM_DEVICE_ERROR;
}

int qmm_gguf_load_entries(const qmm_gguf* g, int64_t i, int64_t count, const int64_t* slots, void* dst,
                          size_t dst_bytes, int64_t stream) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size() || !dst || count < 0 || (count > 0 && !slots))
    return QMM_UNSUPPORTED;
  const Tensor& t = g->tensors[i];
  int64_t bs = 0, ts = 0;
  if (!t.whole || t.n_dims < 2 || t.dims[0] <= 0 || !type_shape(t.type, bs, ts)) return QMM_UNSUPPORTED;
  const int64_t entries = t.dims[0];
  const int64_t per = t.nelem / entries;  // values of one entry
  if (per % bs) return QMM_UNSUPPORTED;   // an entry is a whole number of blocks
  const uint64_t eb = (uint64_t)(per / bs * ts);
  const size_t padded = qmm_padded_bytes(t.type, t.nelem);
  if (padded == 0) return QMM_UNSUPPORTED;
  if (dst_bytes < padded) return QMM_WORKSPACE_TOO_SMALL;
  for (int64_t c = 0; c < count; c++)
    if (slots[c] < 0 || slots[c] >= entries) return QMM_UNSUPPORTED;  // nothing copied
  uint64_t base = 0;
  if (!tensor_span(g, t, base)) return QMM_UNSUPPORTED;
  const hipStream_t st = (hipStream_t)stream;
  std::lock_guard<std::mutex> lock(g_staging.mu);
  (void)hipGetLastError();
  uint8_t* d = (uint8_t*)dst;
  // every slot not named stays zero, as does the padding
  if (hipMemsetAsync(d, 0, padded, st) != hipSuccess) return QMM_DEVICE_ERROR;
  int rc = QMM_OK;
  for (int64_t c = 0; c < count && rc == QMM_OK; c++)
    rc = copy_span(g->fd, base + (uint64_t)slots[c] * eb, eb, d + (uint64_t)slots[c] * eb, st);
  const bool synced = hipStreamSynchronize(st) == hipSuccess;
  if (rc != QMM_OK) return rc;
  return synced ? QMM_OK : QMM_DEVICE_ERROR;
}

int qmm_load_entries(int type, int64_t entries, size_t entry_bytes, int64_t count, const int64_t* slots,
                     const void* const* parts, void* dst, size_t dst_bytes, int64_t stream) {
  int64_t bs = 0, ts = 0;
  if (!type_shape(type, bs, ts) || entries < 0 || count < 0 || !dst || (count > 0 && (!slots || !parts)))
    return QMM_UNSUPPORTED;
  if (entry_bytes % (size_t)ts) return QMM_UNSUPPORTED;  // whole blocks
  if (entries > 0 && entry_bytes > (size_t)(INT64_MAX - pad_bytes(bs, ts)) / (size_t)entries) return QMM_UNSUPPORTED;
  const size_t len = (size_t)entries * entry_bytes, padded = len + (size_t)pad_bytes(bs, ts);
  if (dst_bytes < padded) return QMM_WORKSPACE_TOO_SMALL;
  for (int64_t c = 0; c < count; c++)
    if (slots[c] < 0 || slots[c] >= entries || (entry_bytes && !parts[c])) return QMM_UNSUPPORTED;  // nothing copied
  const hipStream_t st = (hipStream_t)stream;
  (void)hipGetLastError();
  uint8_t* d = (uint8_t*)dst;
  if (hipMemsetAsync(d, 0, padded, st) != hipSuccess) return QMM_DEVICE_ERROR;
  for (int64_t c = 0; c < count; c++)
    if (entry_bytes &&
        hipMemcpyAsync(d + (size_t)slots[c] * entry_bytes, parts[c], entry_bytes, hipMemcpyHostToDevice, st) !=
            hipSuccess)
      return QMM_DEVICE_ERROR;
  // the parts may be released when this returns
  return hipStreamSynchronize(st) == hipSuccess ? QMM_OK : QMM_DEVICE_ERROR;
}

int qmm_load_beside(int type, const void* data, size_t len, void* dst, size_t dst_bytes, int64_t copy_stream,
                    int64_t stream) {
  int64_t bs = 0, ts = 0;
  if (!type_shape(type, bs, ts) || !dst || (len && !data) || len % (size_t)ts) return QMM_UNSUPPORTED;
  if (len > (size_t)(INT64_MAX - pad_bytes(bs, ts))) return QMM_UNSUPPORTED;
  const size_t padded = len + (size_t)pad_bytes(bs, ts);
  if (dst_bytes < padded) return QMM_WORKSPACE_TOO_SMALL;
  const hipStream_t cs = (hipStream_t)copy_stream, st = (hipStream_t)stream;
  (void)hipGetLastError();
  uint8_t* d = (uint8_t*)dst;
  hipEvent_t ev = nullptr;
  if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return QMM_DEVICE_ERROR;
  bool ok = (len == 0 || hipMemcpyAsync(d, data, len, hipMemcpyHostToDevice, cs) == hipSuccess) &&
            hipMemsetAsync(d + len, 0, padded - len, cs) == hipSuccess && hipEventRecord(ev, cs) == hipSuccess &&
            hipStreamWaitEvent(st, ev, 0) == hipSuccess;
  // the host bytes may be released when this returns: wait for the copy
  // alone (work queued on `stream` keeps running meanwhile)
  ok = hipEventSynchronize(ev) == hipSuccess && ok;
  (void)hipEventDestroy(ev);
  return ok ? QMM_OK : QMM_DEVICE_ERROR;
}

}  // extern "C"
