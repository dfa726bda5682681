// C ABI of libstrata_hip: context, resident weight store, entry points.
//
// Host-side mirror of the reference's device backend behaviour
// (crates/strata-backend-wgpu/src/gpu.rs): a name-keyed weight cache
// bounded by a byte budget with least-recently-used eviction (gpu.rs:61-113),
// reusable scratch buffers grown on demand (gpu.rs:126-150,244-262), one lock
// per context (gpu.rs:122-124). Unlike the wgpu backend the weights are
// uploaded packed (GGUF blocks), not dequantized to f32 on the host.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/strata_hip.h"
#include "common.hpp"
#include "gguf.hpp"
#include "kernels.hpp"
#include "store.hpp"

// Device scratch of the allocation-free entry point (sh_ffn_dev_noalloc):
// a fixed array in the library's code object, so using it allocates
// nothing. Each device holds its own copy until the process ends. Host code
// never passes `scratch` itself (a host-side name, not a device address):
// it passes the per-device address from hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local std::string t_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory) return fail(SH_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
    return fail(SH_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return fail(SH_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                  \
  do {                                       \
    hipError_t e_ = (expr);                  \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// Per-device addresses of `scratch` (hipGetSymbolAddress, once per device).
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];

struct Resident {
  void* dev = nullptr;
  uint64_t bytes = 0;
  uint64_t used = 0;
  uint64_t pin = 0;  // the call that last admitted or hit it (never evicted by that call)
  uint32_t quant = 0;
  uint64_t rows = 0, cols = 0, n_expert = 0;
};

// A device buffer that only grows.
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  int ensure(size_t need, const char* what) {
    if (need <= cap && p) return SH_OK;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    size_t sz = (need + 4095) & ~size_t(4095);
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      p = nullptr;
      return hip_fail(e, what);
    }
    cap = sz;
    return SH_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
};

// Pinned host staging (hipHostMalloc: page-locked, allocated as such),
// mapped into the device's address space and coherent (device accesses are
// not cached), so kernels read a call's inputs from it and write its outputs
// to it directly: `dev` is the device's address of `p`.
struct HostBuf {
  void* p = nullptr;
  void* dev = nullptr;
  size_t cap = 0;
  int ensure(size_t need, const char* what) {
    if (need <= cap && p) return SH_OK;
    release();
    size_t sz = (need + 4095) & ~size_t(4095);
    hipError_t e = hipHostMalloc(&p, sz, hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) {
      p = nullptr;
      return hip_fail(e, what);
    }
    e = hipHostGetDevicePointer(&dev, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      p = dev = nullptr;
      return hip_fail(e, what);
    }
    cap = sz;
    return SH_OK;
  }
  void release() {
    if (p) (void)hipHostFree(p);
    p = dev = nullptr;
    cap = 0;
  }
};

}  // namespace

struct sh_context {
  int device = 0;
  hipStream_t stream = nullptr;
  uint64_t budget = 0;
  uint64_t bytes = 0;
  uint64_t clock = 0;
  uint64_t call = 0;  // numbers the locked calls; admissions pin their entry to it
  std::unordered_map<uint64_t, Resident> weights;
  DevBuf d_in, d_out, d_blk;
  HostBuf h_in, h_out;
  HostBuf stage[2];                      // pinned chunks of weight uploads
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  std::mutex mu;
};

namespace {

void free_resident(Resident& r) {
  if (r.dev) (void)hipFree(r.dev);
  r.dev = nullptr;
}

// Copies n host bytes (e.g. an mmap'd GGUF payload, which is pageable) to
// device memory through two pinned 16 MiB chunks: the host copy into one
// chunk (split over kStageThreads threads: one thread's memcpy runs at about
// half the DMA rate) overlaps the DMA out of the other. Synchronous.
constexpr size_t kStageChunk = size_t(16) << 20;
constexpr int kStageThreads = 4;

void parallel_copy(uint8_t* dst, const uint8_t* src, size_t n) {
  if (n < (size_t(1) << 20)) {
    memcpy(dst, src, n);
    return;
  }
  const size_t part = (n / kStageThreads + 4095) & ~size_t(4095);
  std::thread t[kStageThreads - 1];
  int started = 1;  // parts [0, started) are copied by this thread or a helper
  try {
    for (; started < kStageThreads; ++started) {
      const size_t a = std::min(n, part * started), b = std::min(n, part * (started + 1));
      t[started - 1] = std::thread([=] { memcpy(dst + a, src + a, b - a); });
    }
  } catch (const std::exception&) {
    // no thread to be had: the parts not handed out are copied here
  }
  memcpy(dst, src, std::min(n, part));
  const size_t rest = std::min(n, part * started);
  if (rest < n) memcpy(dst + rest, src + rest, n - rest);
  for (int i = 1; i < started; ++i) t[i - 1].join();
}

int staged_upload(sh_context* c, void* dev, const uint8_t* src, uint64_t n) {
  for (int b = 0; b < 2; ++b) {
    int rc = c->stage[b].ensure(kStageChunk, "upload staging");
    if (rc) return rc;
    if (!c->stage_done[b]) HIP_TRY(hipEventCreateWithFlags(&c->stage_done[b], hipEventDisableTiming), "event");
  }
  uint8_t* d = static_cast<uint8_t*>(dev);
  int k = 0;
  for (uint64_t off = 0; off < n; off += kStageChunk, ++k) {
    const int b = k & 1;
    const size_t len = size_t(std::min<uint64_t>(kStageChunk, n - off));
    if (k >= 2) HIP_TRY(hipEventSynchronize(c->stage_done[b]), "upload staging wait");  // chunk b is free
    parallel_copy(static_cast<uint8_t*>(c->stage[b].p), src + off, len);
    HIP_TRY(hipMemcpyAsync(d + off, c->stage[b].p, len, hipMemcpyHostToDevice, c->stream), "weight upload");
    HIP_TRY(hipEventRecord(c->stage_done[b], c->stream), "event");
  }
  HIP_TRY(hipStreamSynchronize(c->stream), "weight upload");
  return SH_OK;
}

// Evicts least-recently-used entries until `incoming` more bytes fit, or the
// store is empty (gpu.rs:88-112): a single tensor larger than the budget is
// still admitted, alone. Entries the current call has admitted are never
// evicted (sh::plan_eviction); when they keep the store over budget the
// admission fails with SH_ERR_OUT_OF_MEMORY and nothing is evicted.
int make_room(sh_context* c, uint64_t key, uint64_t incoming) {
  std::vector<sh::StoreEntry> entries;
  entries.reserve(c->weights.size());
  for (const auto& kv : c->weights) entries.push_back({kv.first, kv.second.bytes, kv.second.used, kv.second.pin});
  std::vector<uint64_t> victims;
  if (!sh::plan_eviction(entries, c->bytes, c->budget, incoming, c->call, &victims))
    return fail(SH_ERR_OUT_OF_MEMORY,
                "weight %llu (%llu bytes): the budget of %llu bytes does not hold it beside the %llu bytes "
                "this call already uses",
                (unsigned long long)key, (unsigned long long)incoming, (unsigned long long)c->budget,
                (unsigned long long)c->bytes);
  for (uint64_t v : victims) {
    auto it = c->weights.find(v);
    c->bytes -= it->second.bytes;
    free_resident(it->second);
    c->weights.erase(it);
  }
  return SH_OK;
}

// The device copy of a weight, uploading the packed bytes on first use. The
// entry is pinned to the current call: later admissions of the same call do
// not evict it, so every pointer a call has obtained stays valid until it
// returns.
int resident(sh_context* c, uint64_t key, uint32_t quant, uint64_t n_expert, uint64_t rows,
             uint64_t cols, const uint8_t* data, uint64_t nbytes, Resident** out) {
  auto it = c->weights.find(key);
  if (it != c->weights.end()) {
    Resident& r = it->second;
    if (r.quant == quant && r.rows == rows && r.cols == cols && r.n_expert == n_expert &&
        r.bytes == nbytes) {
      r.used = ++c->clock;
      r.pin = c->call;
      *out = &r;
      return SH_OK;
    }
    if (r.pin == c->call)  // replacing it would free memory this call holds
      return fail(SH_ERR_INVALID_ARGUMENT, "weight key %llu names two different tensors in one call",
                  (unsigned long long)key);
    // same key, different tensor: replace it
    c->bytes -= r.bytes;
    free_resident(r);
    c->weights.erase(it);
  }
  if (!data) return fail(SH_ERR_INVALID_ARGUMENT, "weight %llu: null data", (unsigned long long)key);
  int rc = make_room(c, key, nbytes);
  if (rc) return rc;
  Resident r;
  r.quant = quant;
  r.rows = rows;
  r.cols = cols;
  r.n_expert = n_expert;
  r.bytes = nbytes;
  hipError_t e = hipMalloc(&r.dev, nbytes ? nbytes : 1);
  if (e != hipSuccess) return hip_fail(e, "uploading weight");
  rc = staged_upload(c, r.dev, data, nbytes);
  if (rc != SH_OK) {
    (void)hipFree(r.dev);
    return rc;
  }
  r.used = ++c->clock;
  r.pin = c->call;
  c->bytes += nbytes;
  auto ins = c->weights.emplace(key, r);
  *out = &ins.first->second;
  return SH_OK;
}

// Shape checks shared by the matrix entry points; mirrors what the
// reference asserts (ops.rs:15-17) or reports (dequant.rs:50-55).
// `matvec`: the entry point runs on the matvec kernels, which also take
// F32 / F16 / BF16 and Q5_K.
int check_matrix(uint32_t quant, uint64_t rows, uint64_t cols, uint64_t n_expert, uint64_t nbytes,
                 bool matvec = false) {
  sh::Geometry g = sh::geometry(quant);
  if (g.block == 0) return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u is not supported", quant);
  if (!sh::device_quant(quant) && !(matvec && (sh::plain_quant(quant) || sh::gemv_quant(quant))))
    return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u has no device kernel here", quant);
  if (cols % uint64_t(g.block) != 0)
    return fail(SH_ERR_TRUNCATED, "cols %llu is not a whole number of %lld-element blocks",
                (unsigned long long)cols, (long long)g.block);
  uint64_t need = 0;
  if (__builtin_mul_overflow(n_expert, rows, &need) ||
      __builtin_mul_overflow(need, cols / uint64_t(g.block), &need) ||
      __builtin_mul_overflow(need, uint64_t(g.bytes), &need))
    return fail(SH_ERR_INVALID_ARGUMENT, "tensor of %llu x %llu x %llu elements: byte size overflows 64 bits",
                (unsigned long long)n_expert, (unsigned long long)rows, (unsigned long long)cols);
  if (nbytes < need)
    return fail(SH_ERR_TRUNCATED, "%llu bytes for a tensor that needs %llu", (unsigned long long)nbytes,
                (unsigned long long)need);
  return SH_OK;
}

// The alternate reading a kernel applies to a tensor's blocks (each type has
// at most one): Q6_K's int8 sub-block scales, or IQ4_XS's ggml qs layout.
static int reading(uint32_t quant, uint32_t flags) {
  if (quant == SH_QUANT_Q6_K) return (flags & SH_FLAG_Q6K_SIGNED_SCALES) ? 1 : 0;
  if (quant == SH_QUANT_IQ4_XS) return (flags & SH_FLAG_IQ4XS_GGML) ? 1 : 0;
  return 0;
}

// Holds the context lock for one call and numbers the call, so the weights
// it admits are pinned until it returns.
struct Guard {
  sh_context* c;
  std::lock_guard<std::mutex> lk;
  explicit Guard(sh_context* ctx) : c(ctx), lk(ctx->mu) { ++c->call; }
};

}  // namespace

extern "C" {

int sh_abi_version(void) { return SH_ABI_VERSION; }

const char* sh_last_error(void) { return t_error.c_str(); }

int sh_device_count(int* count) {
  if (!count) return fail(SH_ERR_INVALID_ARGUMENT, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) n = 0;
  else if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  return SH_OK;
}

int sh_quant_geometry(uint32_t quant, uint32_t* block_size, uint32_t* type_size) {
  sh::Geometry g = sh::geometry(quant);
  if (g.block == 0) return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u is not supported", quant);
  if (block_size) *block_size = uint32_t(g.block);
  if (type_size) *type_size = uint32_t(g.bytes);
  return SH_OK;
}

int sh_create(int device, uint64_t weight_budget_bytes, sh_context** out) {
  if (!out) return fail(SH_ERR_INVALID_ARGUMENT, "null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(SH_ERR_NO_DEVICE, "no HIP device available");
  if (device < 0 || device >= n)
    return fail(SH_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, n);
  HIP_TRY(hipSetDevice(device), "hipSetDevice");
  sh_context* c = new sh_context();
  c->device = device;
  c->budget = weight_budget_bytes ? weight_budget_bytes : (uint64_t(4) << 30);
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreate");
  }
  *out = c;
  return SH_OK;
}

int sh_destroy(sh_context* c) {
  if (!c) return SH_OK;
  {
    std::lock_guard<std::mutex> lk(c->mu);
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (auto& kv : c->weights) free_resident(kv.second);
    c->weights.clear();
    c->d_in.release();
    c->d_out.release();
    c->d_blk.release();
    c->h_in.release();
    c->h_out.release();
    for (int b = 0; b < 2; ++b) {
      c->stage[b].release();
      if (c->stage_done[b]) (void)hipEventDestroy(c->stage_done[b]);
    }
    (void)hipStreamDestroy(c->stream);
  }
  delete c;
  return SH_OK;
}

const char* sh_name(const sh_context*) { return "hip"; }

int sh_resident_bytes(sh_context* c, uint64_t* bytes) {
  if (!c || !bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lk(c->mu);
  *bytes = c->bytes;
  return SH_OK;
}

int sh_evict(sh_context* c, uint64_t key) {
  if (!c) return fail(SH_ERR_INVALID_ARGUMENT, "null context");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->weights.find(key);
  if (it != c->weights.end()) {
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    c->bytes -= it->second.bytes;
    free_resident(it->second);
    c->weights.erase(it);
  }
  return SH_OK;
}

// Host x -> device, kernel, host y; all on the context stream. The matvec
// kernels only store y, so they write it straight into the mapped staging
// (one 4-byte store per row: measured +0.2 us against device memory, where a
// copy kernel back would add about 2 us).
static int run_gemv(sh_context* c, const sh_quant_tensor* w, const float* x, float* y,
                    uint32_t batch) {
  const uint64_t rows = w->rows, cols = w->cols;
  if (rows == 0) return SH_OK;
  if (cols == 0) {  // ops::gemv: every row sums nothing
    memset(y, 0, sizeof(float) * rows * batch);
    return SH_OK;
  }
  if (!sh::gemv_shape_ok(w->quant, int64_t(rows), int64_t(cols), int(batch)))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "gemv %llux%llu of type %u (batch %u) is not supported",
                (unsigned long long)rows, (unsigned long long)cols, w->quant, batch);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident* r = nullptr;
  const uint64_t need = rows * uint64_t(sh::byte_size(w->quant, int64_t(cols)));
  int rc = resident(c, w->key, w->quant, 1, rows, cols, w->data, need, &r);
  if (rc) return rc;
  const size_t xb = sizeof(float) * cols * batch, yb = sizeof(float) * rows * batch;
  if ((rc = c->d_in.ensure(xb, "x buffer")) || (rc = c->h_in.ensure(xb, "x staging")) ||
      (rc = c->h_out.ensure(yb, "y staging")))
    return rc;
  const size_t wsb = sh::gemv_workspace_bytes(w->quant, int64_t(rows), int64_t(cols), int(batch));
  if (wsb && (rc = c->d_blk.ensure(wsb, "workspace"))) return rc;
  memcpy(c->h_in.p, x, xb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, xb, c->stream), "x upload");
  HIP_TRY(sh::launch_gemv(w->quant, r->dev, int64_t(rows), int64_t(cols),
                          static_cast<const float*>(c->d_in.p), static_cast<float*>(c->h_out.dev),
                          int(batch), reading(w->quant, w->flags), c->stream,
                          wsb ? c->d_blk.p : nullptr),
          "gemv launch");
  HIP_TRY(hipStreamSynchronize(c->stream), "gemv");
  memcpy(y, c->h_out.p, yb);
  return SH_OK;
}

int sh_gemv(sh_context* c, const sh_quant_tensor* w, const float* x, uint64_t x_len, float* y,
            uint64_t y_len) {
  if (!c || !w || (!x && x_len) || (!y && y_len)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (x_len != w->cols) return fail(SH_ERR_SHAPE, "gemv: x has %llu elements, cols is %llu",
                                    (unsigned long long)x_len, (unsigned long long)w->cols);
  if (y_len != w->rows) return fail(SH_ERR_SHAPE, "gemv: y has %llu elements, rows is %llu",
                                    (unsigned long long)y_len, (unsigned long long)w->rows);
  int rc = check_matrix(w->quant, w->rows, w->cols, 1, w->nbytes, true);
  if (rc) return rc;
  Guard g(c);
  return run_gemv(c, w, x, y, 1);
}

int sh_gemv_batch(sh_context* c, const sh_quant_tensor* w, const float* x, float* y, uint32_t batch) {
  if (!c || !w || !x || !y) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (batch < 1 || batch > 8) return fail(SH_ERR_INVALID_ARGUMENT, "batch %u is outside 1..8", batch);
  int rc = check_matrix(w->quant, w->rows, w->cols, 1, w->nbytes, true);
  if (rc) return rc;
  Guard g(c);
  return run_gemv(c, w, x, y, batch);
}

int sh_expert_gemv(sh_context* c, const sh_expert_view* w, uint64_t e, const float* x,
                   uint64_t x_len, float* y, uint64_t y_len) {
  if (!c || !w || (!x && x_len) || (!y && y_len)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (w->flags & SH_FLAG_EXPERT_OUT_MAJOR) {
    // ggml orientation: expert e is an ordinary [rows = out][cols = in]
    // matrix, run by the matvec kernels on its slice of the resident stack
    if (x_len != w->cols) return fail(SH_ERR_SHAPE, "expert_gemv: x has %llu elements, cols is %llu",
                                      (unsigned long long)x_len, (unsigned long long)w->cols);
    if (y_len != w->rows) return fail(SH_ERR_SHAPE, "expert_gemv: y has %llu elements, rows is %llu",
                                      (unsigned long long)y_len, (unsigned long long)w->rows);
    if (e >= w->n_expert) return fail(SH_ERR_SHAPE, "expert %llu of %llu", (unsigned long long)e,
                                      (unsigned long long)w->n_expert);
    int rc = check_matrix(w->quant, w->rows, w->cols, w->n_expert, w->nbytes, true);
    if (rc) return rc;
    const uint64_t rows = w->rows, cols = w->cols;
    if (rows == 0) return SH_OK;
    if (cols == 0) {
      memset(y, 0, sizeof(float) * rows);
      return SH_OK;
    }
    if (!sh::gemv_shape_ok(w->quant, int64_t(rows), int64_t(cols), 1))
      return fail(SH_ERR_UNSUPPORTED_SHAPE, "expert_gemv %llux%llu of type %u is not supported",
                  (unsigned long long)rows, (unsigned long long)cols, w->quant);
    Guard g(c);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    Resident* r = nullptr;
    const uint64_t rb = uint64_t(sh::byte_size(w->quant, int64_t(cols)));
    rc = resident(c, w->key, w->quant, w->n_expert, rows, cols, w->data, w->n_expert * rows * rb, &r);
    if (rc) return rc;
    const size_t xb = sizeof(float) * cols, yb = sizeof(float) * rows;
    if ((rc = c->d_in.ensure(xb, "x buffer")) || (rc = c->h_in.ensure(xb, "x staging")) ||
        (rc = c->h_out.ensure(yb, "y staging")))
      return rc;
    const uint8_t* we = static_cast<const uint8_t*>(r->dev) + e * rows * rb;
    memcpy(c->h_in.p, x, xb);
    HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, xb, c->stream), "x upload");
    HIP_TRY(sh::launch_gemv(w->quant, we, int64_t(rows), int64_t(cols), static_cast<const float*>(c->d_in.p),
                            static_cast<float*>(c->h_out.dev), 1, reading(w->quant, w->flags),
                            c->stream),
            "expert_gemv launch");  // y straight into the mapped staging, as run_gemv
    HIP_TRY(hipStreamSynchronize(c->stream), "expert_gemv");
    memcpy(y, c->h_out.p, yb);
    return SH_OK;
  }
  if (x_len != w->rows) return fail(SH_ERR_SHAPE, "expert_gemv: x has %llu elements, rows is %llu",
                                    (unsigned long long)x_len, (unsigned long long)w->rows);
  if (y_len != w->cols) return fail(SH_ERR_SHAPE, "expert_gemv: y has %llu elements, cols is %llu",
                                    (unsigned long long)y_len, (unsigned long long)w->cols);
  if (e >= w->n_expert) return fail(SH_ERR_SHAPE, "expert %llu of %llu", (unsigned long long)e,
                                    (unsigned long long)w->n_expert);
  int rc = check_matrix(w->quant, w->rows, w->cols, w->n_expert, w->nbytes);
  if (rc) return rc;
  const uint64_t rows = w->rows, cols = w->cols;
  if (cols == 0) return SH_OK;
  if (rows == 0) {  // ops::expert_gemv: no input rows, all sums zero
    memset(y, 0, sizeof(float) * cols);
    return SH_OK;
  }
  if (!sh::expert_shape_ok(w->quant, int64_t(rows), int64_t(cols)))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "expert_gemv %llux%llu of type %u is not supported",
                (unsigned long long)rows, (unsigned long long)cols, w->quant);
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident* r = nullptr;
  const uint64_t need = w->n_expert * rows * uint64_t(sh::byte_size(w->quant, int64_t(cols)));
  rc = resident(c, w->key, w->quant, w->n_expert, rows, cols, w->data, need, &r);
  if (rc) return rc;
  const size_t xb = sizeof(float) * rows, yb = sizeof(float) * cols;
  const size_t ws = sh::expert_workspace_bytes(int64_t(rows), int64_t(cols));
  if ((rc = c->d_in.ensure(xb, "x buffer")) || (rc = c->d_blk.ensure(ws, "workspace")) ||
      (rc = c->h_in.ensure(xb, "x staging")) || (rc = c->h_out.ensure(yb, "y staging")))
    return rc;
  const uint8_t* we = static_cast<const uint8_t*>(r->dev) +
                      e * rows * uint64_t(sh::byte_size(w->quant, int64_t(cols)));
  memcpy(c->h_in.p, x, xb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, xb, c->stream), "x upload");
  // the column sums store y once per column: straight into the mapped staging
  HIP_TRY(sh::launch_expert_gemv(w->quant, we, int64_t(rows), int64_t(cols),
                                 static_cast<const float*>(c->d_in.p), static_cast<float*>(c->h_out.dev),
                                 static_cast<float*>(c->d_blk.p),
                                 reading(w->quant, w->flags), c->stream),
          "expert_gemv launch");
  HIP_TRY(hipStreamSynchronize(c->stream), "expert_gemv");
  memcpy(y, c->h_out.p, yb);
  return SH_OK;
}

// The orientation of a call's three expert stacks: 0 all in-major (the
// reference's [n_expert][in][out]), 1 all out-major (SH_FLAG_EXPERT_OUT_MAJOR,
// llama.cpp's [n_expert][out][in]), -1 mixed.
static int orientation(uint32_t fg, uint32_t fu, uint32_t fd) {
  const uint32_t a = fg & SH_FLAG_EXPERT_OUT_MAJOR, b = fu & SH_FLAG_EXPERT_OUT_MAJOR,
                 d = fd & SH_FLAG_EXPERT_OUT_MAJOR;
  if (a != b || b != d) return -1;
  return a ? 1 : 0;
}

static int mixed_orientation() {
  return fail(SH_ERR_UNSUPPORTED_SHAPE, "gate, up and down must share one orientation (SH_FLAG_EXPERT_OUT_MAJOR)");
}

static int moe_check(uint64_t n_expert, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok,
                     uint32_t top_k, uint32_t qa, uint32_t qb, sh::MoePlan* plan, bool out_major = false) {
  if (n_expert == 0 || n_expert > uint64_t(sh::kMoeMaxExperts))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "n_expert %llu outside 1..%d", (unsigned long long)n_expert,
                sh::kMoeMaxExperts);
  if (top_k == 0 || top_k > uint32_t(sh::kMoeMaxTopK) || top_k > n_expert)
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "top_k %u outside 1..min(%d, n_expert)", top_k, sh::kMoeMaxTopK);
  if (n_tok == 0 || n_tok > uint32_t(sh::kMoeMaxTokens))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "n_tok %u outside 1..%d", n_tok, sh::kMoeMaxTokens);
  if (n_embd > (1u << 20) || n_ff > (1u << 20))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "MoE widths too large");
  if (!sh::moe_plan(int(n_tok), int(top_k), int(n_expert), int(n_embd), int(n_ff), qa, qb, plan, out_major))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "MoE %llu x %llu (types %u, %u, %s) is not supported",
                (unsigned long long)n_embd, (unsigned long long)n_ff, qa, qb, out_major ? "out-major" : "in-major");
  return SH_OK;
}

int sh_moe_route(sh_context* c, const float* logits, uint32_t n_tok, uint32_t n_expert, uint32_t top_k,
                 int32_t* ids, float* weights) {
  if (!c || !logits || !ids || !weights) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  sh::MoePlan plan;
  // routing needs no weights: plan with a minimal Q4_K shape for the layout
  int rc = moe_check(n_expert, 256, 256, n_tok, top_k, sh::kQ4_K, sh::kQ4_K, &plan);
  if (rc) return rc;
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  const size_t lb = sizeof(float) * n_tok * n_expert, ob = sizeof(float) * n_tok * top_k;
  if ((rc = c->d_in.ensure(lb, "logits buffer")) || (rc = c->d_blk.ensure(plan.bytes, "workspace")) ||
      (rc = c->h_in.ensure(lb, "logits staging")) || (rc = c->h_out.ensure(2 * ob, "route staging")))
    return rc;
  memcpy(c->h_in.p, logits, lb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, lb, c->stream), "logits upload");
  HIP_TRY(sh::launch_moe_route(plan, static_cast<const float*>(c->d_in.p), c->d_blk.p, c->stream), "route");
  uint8_t* ho = static_cast<uint8_t*>(c->h_out.p);
  const uint8_t* blk = static_cast<const uint8_t*>(c->d_blk.p);
  HIP_TRY(sh::launch_copy_bytes(blk + plan.o_ids, c->h_out.dev, ob, c->stream), "ids readback");
  HIP_TRY(sh::launch_copy_bytes(blk + plan.o_wts, static_cast<uint8_t*>(c->h_out.dev) + ob, ob, c->stream),
          "weights readback");
  HIP_TRY(hipStreamSynchronize(c->stream), "route");
  memcpy(ids, ho, ob);
  memcpy(weights, ho + ob, ob);
  return SH_OK;
}

int sh_moe_ffn(sh_context* c, const sh_expert_view* gate, const sh_expert_view* up,
               const sh_expert_view* down, const float* logits, uint32_t n_tok, uint32_t top_k,
               const float* x, float* out) {
  if (!c || !gate || !up || !down || !logits || !x || !out)
    return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const int om = orientation(gate->flags, up->flags, down->flags);
  if (om < 0) return mixed_orientation();
  // gate / up [E][gr][gc], down [E][gc][gr] in either orientation:
  // (gr, gc) = (n_embd, n_ff) in-major, (n_ff, n_embd) out-major
  const uint64_t E = gate->n_expert, gr = gate->rows, gc = gate->cols;
  const uint64_t n_embd = om ? gc : gr, n_ff = om ? gr : gc;
  if (up->n_expert != E || down->n_expert != E || up->rows != gr || up->cols != gc || down->rows != gc ||
      down->cols != gr)
    return fail(SH_ERR_SHAPE, "MoE views disagree: gate/up [%llu][%llu][%llu], down [%llu][%llu][%llu]",
                (unsigned long long)E, (unsigned long long)gr, (unsigned long long)gc,
                (unsigned long long)down->n_expert, (unsigned long long)down->rows,
                (unsigned long long)down->cols);
  if (gate->quant != up->quant)
    return fail(SH_ERR_UNSUPPORTED_QUANT, "gate (%u) and up (%u) types differ", gate->quant, up->quant);
  int rc;
  if ((rc = check_matrix(gate->quant, gr, gc, E, gate->nbytes)) ||
      (rc = check_matrix(up->quant, gr, gc, E, up->nbytes)) ||
      (rc = check_matrix(down->quant, gc, gr, E, down->nbytes)))
    return rc;
  sh::MoePlan plan;
  if ((rc = moe_check(E, n_embd, n_ff, n_tok, top_k, gate->quant, down->quant, &plan, om == 1))) return rc;
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident *rg = nullptr, *ru = nullptr, *rd = nullptr;
  const uint64_t ga = E * gr * uint64_t(sh::byte_size(gate->quant, int64_t(gc)));
  const uint64_t db = E * gc * uint64_t(sh::byte_size(down->quant, int64_t(gr)));
  if ((rc = resident(c, gate->key, gate->quant, E, gr, gc, gate->data, ga, &rg))) return rc;
  if ((rc = resident(c, up->key, up->quant, E, gr, gc, up->data, ga, &ru))) return rc;
  if ((rc = resident(c, down->key, down->quant, E, gc, gr, down->data, db, &rd))) return rc;
  const size_t lb = sizeof(float) * n_tok * E, xb = sizeof(float) * n_tok * n_embd;
  const size_t lb_al = (lb + 255) & ~size_t(255);
  if ((rc = c->d_in.ensure(lb_al + xb, "inputs")) || (rc = c->d_out.ensure(xb, "out buffer")) ||
      (rc = c->d_blk.ensure(plan.bytes, "workspace")) || (rc = c->h_in.ensure(lb_al + xb, "staging")) ||
      (rc = c->h_out.ensure(xb, "out staging")))
    return rc;
  uint8_t* hi = static_cast<uint8_t*>(c->h_in.p);
  memcpy(hi, logits, lb);
  memcpy(hi + lb_al, x, xb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, lb_al + xb, c->stream), "input upload");
  const uint8_t* di = static_cast<const uint8_t*>(c->d_in.p);
  HIP_TRY(sh::launch_moe(plan, gate->quant, up->quant, down->quant, rg->dev, ru->dev, rd->dev,
                         reading(gate->quant, gate->flags),
                         reading(up->quant, up->flags),
                         reading(down->quant, down->flags),
                         reinterpret_cast<const float*>(di), reinterpret_cast<const float*>(di + lb_al),
                         static_cast<float*>(c->d_out.p), c->d_blk.p, c->stream),
          "moe launch");
  HIP_TRY(sh::launch_copy_bytes(c->d_out.p, c->h_out.dev, xb, c->stream), "out readback");
  HIP_TRY(hipStreamSynchronize(c->stream), "moe");
  memcpy(out, c->h_out.p, xb);
  return SH_OK;
}

// The layer's dense tensors against the routed views: router [n_expert][n_embd],
// gate/up_shexp [n_ff_sh][n_embd], down_shexp [n_embd][n_ff_sh],
// gate_inp_shexp [1][n_embd]; then the plan.
static int moe_layer_check(uint64_t E, uint64_t n_embd, uint64_t n_ff, uint64_t n_sh, uint32_t n_tok,
                           uint32_t top_k, const sh::MoeLayerTypes& q, sh::MoeLayerPlan* plan,
                           bool out_major = false) {
  int rc = moe_check(E, n_embd, n_ff, n_tok, top_k, q.gate, q.down, &plan->moe, out_major);
  if (rc) return rc;
  if (q.up != q.gate)
    return fail(SH_ERR_UNSUPPORTED_QUANT, "gate (%u) and up (%u) types differ", q.gate, q.up);
  if (n_sh == 0 || n_sh > (1u << 20)) return fail(SH_ERR_UNSUPPORTED_SHAPE, "shared expert width %llu",
                                                 (unsigned long long)n_sh);
  if (!sh::moe_layer_plan(int(n_tok), int(top_k), int(E), int(n_embd), int(n_ff), int(n_sh), q, plan, out_major))
    return fail(SH_ERR_UNSUPPORTED_SHAPE,
                "MoE layer: router %llux%llu (type %u) or shared expert %llu wide (types %u, %u, %u, gate %u) "
                "is not a matvec shape the kernels take",
                (unsigned long long)E, (unsigned long long)n_embd, q.router, (unsigned long long)n_sh, q.gate_sh,
                q.up_sh, q.down_sh, q.gate_inp);
  return SH_OK;
}

int sh_moe_layer(sh_context* c, const sh_quant_tensor* router, const sh_expert_view* gate,
                 const sh_expert_view* up, const sh_expert_view* down, const sh_quant_tensor* gate_shexp,
                 const sh_quant_tensor* up_shexp, const sh_quant_tensor* down_shexp,
                 const sh_quant_tensor* gate_inp_shexp, const float* x, uint32_t n_tok, uint32_t top_k,
                 float* out) {
  if (!c || !router || !gate || !up || !down || !gate_shexp || !up_shexp || !down_shexp || !gate_inp_shexp ||
      !x || !out)
    return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const int om = orientation(gate->flags, up->flags, down->flags);
  if (om < 0) return mixed_orientation();
  const uint64_t E = gate->n_expert, gr = gate->rows, gc = gate->cols, n_sh = gate_shexp->rows;
  const uint64_t n_embd = om ? gc : gr, n_ff = om ? gr : gc;
  if (up->n_expert != E || down->n_expert != E || up->rows != gr || up->cols != gc || down->rows != gc ||
      down->cols != gr)
    return fail(SH_ERR_SHAPE, "MoE views disagree: gate/up [%llu][%llu][%llu], down [%llu][%llu][%llu]",
                (unsigned long long)E, (unsigned long long)gr, (unsigned long long)gc,
                (unsigned long long)down->n_expert, (unsigned long long)down->rows,
                (unsigned long long)down->cols);
  if (router->rows != E || router->cols != n_embd || gate_shexp->cols != n_embd || up_shexp->rows != n_sh ||
      up_shexp->cols != n_embd || down_shexp->rows != n_embd || down_shexp->cols != n_sh ||
      gate_inp_shexp->rows != 1 || gate_inp_shexp->cols != n_embd)
    return fail(SH_ERR_SHAPE, "MoE layer: router or shared-expert shapes disagree with the %llu x %llu experts",
                (unsigned long long)E, (unsigned long long)n_embd);
  int rc;
  if ((rc = check_matrix(gate->quant, gr, gc, E, gate->nbytes)) ||
      (rc = check_matrix(up->quant, gr, gc, E, up->nbytes)) ||
      (rc = check_matrix(down->quant, gc, gr, E, down->nbytes)))
    return rc;
  const sh_quant_tensor* dense[5] = {router, gate_shexp, up_shexp, down_shexp, gate_inp_shexp};
  for (const sh_quant_tensor* t : dense)
    if ((rc = check_matrix(t->quant, t->rows, t->cols, 1, t->nbytes, true))) return rc;
  const sh::MoeLayerTypes q{router->quant, gate->quant, up->quant, down->quant,
                            gate_shexp->quant, up_shexp->quant, down_shexp->quant, gate_inp_shexp->quant};
  sh::MoeLayerPlan plan;
  if ((rc = moe_layer_check(E, n_embd, n_ff, n_sh, n_tok, top_k, q, &plan, om == 1))) return rc;
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  // all eight tensors resident at once (each admission is pinned to this
  // call, so a later one cannot evict an earlier one)
  struct Want {
    uint64_t key;
    uint32_t quant;
    uint64_t n_expert, rows, cols;
    const uint8_t* data;
  };
  const Want want[8] = {
      {router->key, router->quant, 1, router->rows, router->cols, router->data},
      {gate->key, gate->quant, E, gr, gc, gate->data},
      {up->key, up->quant, E, gr, gc, up->data},
      {down->key, down->quant, E, gc, gr, down->data},
      {gate_shexp->key, gate_shexp->quant, 1, n_sh, n_embd, gate_shexp->data},
      {up_shexp->key, up_shexp->quant, 1, n_sh, n_embd, up_shexp->data},
      {down_shexp->key, down_shexp->quant, 1, n_embd, n_sh, down_shexp->data},
      {gate_inp_shexp->key, gate_inp_shexp->quant, 1, 1, n_embd, gate_inp_shexp->data}};
  void* dev[8] = {};
  for (int i = 0; i < 8; ++i) {
    Resident* r = nullptr;
    const uint64_t nb = want[i].n_expert * want[i].rows * uint64_t(sh::byte_size(want[i].quant, int64_t(want[i].cols)));
    if ((rc = resident(c, want[i].key, want[i].quant, want[i].n_expert, want[i].rows, want[i].cols,
                       want[i].data, nb, &r)))
      return rc;
    dev[i] = r->dev;
  }
  const size_t xb = sizeof(float) * n_tok * n_embd;
  if ((rc = c->d_in.ensure(xb, "x buffer")) || (rc = c->d_out.ensure(xb, "out buffer")) ||
      (rc = c->d_blk.ensure(plan.bytes, "workspace")) || (rc = c->h_in.ensure(xb, "x staging")) ||
      (rc = c->h_out.ensure(xb, "out staging")))
    return rc;
  memcpy(c->h_in.p, x, xb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, xb, c->stream), "x upload");
  auto q6 = [](const auto* t) { return reading(t->quant, t->flags); };
  const sh::MoeLayerTensors w{dev[0], dev[1], dev[2], dev[3], dev[4], dev[5], dev[6], dev[7],
                              q6(router), q6(gate), q6(up), q6(down),
                              q6(gate_shexp), q6(up_shexp), q6(down_shexp),
                              q6(gate_inp_shexp)};
  HIP_TRY(sh::launch_moe_layer(plan, q, w, static_cast<const float*>(c->d_in.p), static_cast<float*>(c->d_out.p),
                               c->d_blk.p, c->stream),
          "moe layer launch");
  HIP_TRY(sh::launch_copy_bytes(c->d_out.p, c->h_out.dev, xb, c->stream), "out readback");
  HIP_TRY(hipStreamSynchronize(c->stream), "moe layer");
  memcpy(out, c->h_out.p, xb);
  return SH_OK;
}

static int matmul_check(uint32_t quant, uint64_t rows, uint64_t cols, uint64_t m, uint32_t mode) {
  if (mode > SH_MATMUL_Q8K) return fail(SH_ERR_INVALID_ARGUMENT, "matmul mode %u", mode);
  if (!sh::device_quant(quant))
    return fail(SH_ERR_UNSUPPORTED_QUANT, "matmul: type %u has no device kernel", quant);
  if (mode == SH_MATMUL_Q8K && quant != SH_QUANT_Q4_K && quant != SH_QUANT_Q5_K)
    return fail(SH_ERR_UNSUPPORTED_QUANT, "matmul: SH_MATMUL_Q8K takes Q4_K / Q5_K weights only");
  if (!sh::matmul_shape_ok(quant, int64_t(rows), int64_t(cols), int64_t(m), mode))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "matmul %llux%llu (m %llu) of type %u is not supported",
                (unsigned long long)rows, (unsigned long long)cols, (unsigned long long)m, quant);
  return SH_OK;
}

int sh_matmul(sh_context* c, const sh_quant_tensor* w, const float* x, uint32_t m, float* y, uint32_t mode) {
  if (!c || !w || (!x && m) || (!y && m)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = check_matrix(w->quant, w->rows, w->cols, 1, w->nbytes);
  if (rc) return rc;
  const uint64_t rows = w->rows, cols = w->cols;
  if (m == 0 || rows == 0) return SH_OK;
  if (cols == 0) {
    memset(y, 0, sizeof(float) * rows * m);
    return SH_OK;
  }
  if ((rc = matmul_check(w->quant, rows, cols, m, mode))) return rc;
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident* r = nullptr;
  const uint64_t need = rows * uint64_t(sh::byte_size(w->quant, int64_t(cols)));
  if ((rc = resident(c, w->key, w->quant, 1, rows, cols, w->data, need, &r))) return rc;
  const size_t xb = sizeof(float) * cols * m, yb = sizeof(float) * rows * m;
  const size_t ws = sh::matmul_workspace_bytes(int64_t(cols), int64_t(m), mode);
  if ((rc = c->d_in.ensure(xb, "x buffer")) || (rc = c->d_blk.ensure(ws, "workspace")) ||
      (rc = c->h_in.ensure(xb, "x staging")) || (rc = c->h_out.ensure(yb, "y staging")))
    return rc;
  memcpy(c->h_in.p, x, xb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, xb, c->stream), "x upload");
  // the tiles store y once each: straight into the mapped staging
  HIP_TRY(sh::launch_matmul(w->quant, r->dev, int64_t(rows), int64_t(cols),
                            static_cast<const float*>(c->d_in.p), int64_t(m), static_cast<float*>(c->h_out.dev),
                            mode, c->d_blk.p, reading(w->quant, w->flags), c->stream),
          "matmul launch");
  HIP_TRY(hipStreamSynchronize(c->stream), "matmul");
  memcpy(y, c->h_out.p, yb);
  return SH_OK;
}

int sh_dequantize_row(sh_context* c, uint32_t quant, uint32_t flags, const uint8_t* block,
                      uint64_t nbytes, float* out, uint64_t n) {
  if (!c || (!block && nbytes) || (!out && n)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  sh::Geometry g = sh::geometry(quant);
  if (g.block == 0) return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u is not supported", quant);
  const uint64_t nb = (n + uint64_t(g.block) - 1) / uint64_t(g.block);
  if (n % uint64_t(g.block) != 0 || nbytes < nb * uint64_t(g.bytes))
    return fail(SH_ERR_TRUNCATED, "truncated block: expected %llu bytes, found %llu",
                (unsigned long long)(nb * uint64_t(g.bytes)), (unsigned long long)nbytes);
  if (n == 0) return SH_OK;
  Guard gd(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  const size_t in_b = nb * size_t(g.bytes), out_b = sizeof(float) * n;
  int rc;
  if ((rc = c->d_blk.ensure(in_b, "block buffer")) || (rc = c->d_out.ensure(out_b, "out buffer")) ||
      (rc = c->h_out.ensure(out_b, "out staging")))
    return rc;
  HIP_TRY(hipMemcpyAsync(c->d_blk.p, block, in_b, hipMemcpyHostToDevice, c->stream), "block upload");
  HIP_TRY(sh::launch_dequant(quant, c->d_blk.p, 1, int64_t(n), static_cast<float*>(c->d_out.p),
                             reading(quant, flags), c->stream),
          "dequant launch");
  HIP_TRY(sh::launch_copy_bytes(c->d_out.p, c->h_out.dev, out_b, c->stream), "readback");
  HIP_TRY(hipStreamSynchronize(c->stream), "dequant");
  memcpy(out, c->h_out.p, out_b);
  return SH_OK;
}

int sh_dequant_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                   float* out, void* stream) {
  sh::Geometry g = sh::geometry(quant);
  if (g.block == 0) return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u is not supported", quant);
  if (cols % uint64_t(g.block) != 0)
    return fail(SH_ERR_TRUNCATED, "cols %llu is not a whole number of blocks", (unsigned long long)cols);
  if (rows && cols && (!w || !out)) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  HIP_TRY(sh::launch_dequant(quant, w, int64_t(rows), int64_t(cols), out,
                             reading(quant, flags),
                             static_cast<hipStream_t>(stream)),
          "dequant launch");
  return SH_OK;
}

int sh_stream_read_dev(const void* data, uint64_t nbytes, uint32_t* out, void* stream) {
  if ((!data && nbytes) || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if ((reinterpret_cast<uintptr_t>(data) & 15u) || (nbytes & 15u))
    return fail(SH_ERR_INVALID_ARGUMENT, "data must be 16-byte aligned and a multiple of 16 bytes long");
  HIP_TRY(sh::launch_stream_read(data, nbytes, out, static_cast<hipStream_t>(stream)), "stream read launch");
  return SH_OK;
}

int sh_gemv_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                const float* x, float* y, uint32_t batch, void* stream) {
  if (batch < 1 || batch > 8) return fail(SH_ERR_INVALID_ARGUMENT, "batch %u is outside 1..8", batch);
  int rc = check_matrix(quant, rows, cols, 1, ~uint64_t(0), true);
  if (rc) return rc;
  if (rows == 0 || cols == 0)
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "empty matrix on the device path");
  if (!w || !x || !y) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if (!sh::gemv_shape_ok(quant, int64_t(rows), int64_t(cols), int(batch)))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "gemv %llux%llu of type %u (batch %u) is not supported",
                (unsigned long long)rows, (unsigned long long)cols, quant, batch);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 1u) ||
      ((quant == SH_QUANT_Q8_0 || quant == SH_QUANT_F32 || quant == SH_QUANT_IQ4_XS) &&
       (reinterpret_cast<uintptr_t>(w) & 3u)))
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned pointer (w needs 2 bytes, 4 for Q8_0 and F32; x 16)");
  HIP_TRY(sh::launch_gemv(quant, w, int64_t(rows), int64_t(cols), x, y, int(batch),
                          reading(quant, flags), static_cast<hipStream_t>(stream)),
          "gemv launch");
  return SH_OK;
}

int sh_gemv_workspace_bytes(uint32_t quant, uint64_t rows, uint64_t cols, uint32_t batch, uint64_t* bytes) {
  if (!bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null bytes");
  if (batch < 1 || batch > 8) return fail(SH_ERR_INVALID_ARGUMENT, "batch %u is outside 1..8", batch);
  int rc = check_matrix(quant, rows, cols, 1, ~uint64_t(0), true);
  if (rc) return rc;
  if (rows && cols && !sh::gemv_shape_ok(quant, int64_t(rows), int64_t(cols), int(batch)))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "gemv %llux%llu of type %u (batch %u) is not supported",
                (unsigned long long)rows, (unsigned long long)cols, quant, batch);
  *bytes = rows && cols ? sh::gemv_workspace_bytes(quant, int64_t(rows), int64_t(cols), int(batch)) : 0;
  return SH_OK;
}

int sh_gemv_dev_ws(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols, const float* x,
                   float* y, uint32_t batch, void* workspace, uint64_t workspace_bytes, void* stream) {
  uint64_t need = 0;
  int rc = sh_gemv_workspace_bytes(quant, rows, cols, batch, &need);
  if (rc) return rc;
  if (need && (!workspace || workspace_bytes < need))
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace of %llu bytes, %llu needed", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  if (rows == 0 || cols == 0) return fail(SH_ERR_UNSUPPORTED_SHAPE, "empty matrix on the device path");
  if (!w || !x || !y) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 1u) ||
      ((quant == SH_QUANT_Q8_0 || quant == SH_QUANT_F32 || quant == SH_QUANT_IQ4_XS) &&
       (reinterpret_cast<uintptr_t>(w) & 3u)))
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned pointer (w needs 2 bytes, 4 for Q8_0 and F32; x 16)");
  HIP_TRY(sh::launch_gemv(quant, w, int64_t(rows), int64_t(cols), x, y, int(batch),
                          reading(quant, flags), static_cast<hipStream_t>(stream),
                          need ? workspace : nullptr),
          "gemv launch");
  return SH_OK;
}

int sh_moe_workspace_bytes(uint32_t n_tok, uint32_t top_k, uint64_t n_expert, uint64_t n_embd,
                           uint64_t n_ff, uint32_t quant_gate_up, uint32_t quant_down, uint64_t* bytes) {
  if (!bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null bytes");
  // enough for either orientation of the stacks (whichever the shape allows)
  sh::MoePlan in_major, out_major;
  const bool a = sh::moe_plan(int(std::min<uint64_t>(n_tok, 1u << 30)), int(std::min<uint32_t>(top_k, 1u << 30)),
                              int(std::min<uint64_t>(n_expert, 1u << 30)), int(std::min<uint64_t>(n_embd, 1u << 30)),
                              int(std::min<uint64_t>(n_ff, 1u << 30)), quant_gate_up, quant_down, &out_major, true);
  int rc = moe_check(n_expert, n_embd, n_ff, n_tok, top_k, quant_gate_up, quant_down, &in_major);
  if (rc && !a) return rc;
  *bytes = std::max<uint64_t>(rc ? 0 : in_major.bytes, a ? out_major.bytes : 0);
  return SH_OK;
}

int sh_moe_ffn_dev(const sh_expert_dev* gate, const sh_expert_dev* up, const sh_expert_dev* down,
                   uint64_t n_expert, uint64_t n_embd, uint64_t n_ff, const float* logits,
                   uint32_t n_tok, uint32_t top_k, const float* x, float* out, void* workspace,
                   uint64_t workspace_bytes, void* stream) {
  if (!gate || !up || !down || !gate->data || !up->data || !down->data || !logits || !x || !out ||
      !workspace)
    return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const int om = orientation(gate->flags, up->flags, down->flags);
  if (om < 0) return mixed_orientation();
  if (gate->quant != up->quant)
    return fail(SH_ERR_UNSUPPORTED_QUANT, "gate (%u) and up (%u) types differ", gate->quant, up->quant);
  sh::MoePlan plan;
  int rc = moe_check(n_expert, n_embd, n_ff, n_tok, top_k, gate->quant, down->quant, &plan, om == 1);
  if (rc) return rc;
  if (workspace_bytes < plan.bytes)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace of %llu bytes, %llu needed",
                (unsigned long long)workspace_bytes, (unsigned long long)plan.bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  for (const sh_expert_dev* t : {gate, up, down})
    if ((reinterpret_cast<uintptr_t>(t->data) & 1u) ||
        ((t->quant == SH_QUANT_Q8_0 || t->quant == SH_QUANT_IQ4_XS) &&
         (reinterpret_cast<uintptr_t>(t->data) & 3u)))
      return fail(SH_ERR_INVALID_ARGUMENT, "misaligned expert tensor");
  HIP_TRY(sh::launch_moe(plan, gate->quant, up->quant, down->quant, gate->data, up->data, down->data,
                         reading(gate->quant, gate->flags),
                         reading(up->quant, up->flags),
                         reading(down->quant, down->flags), logits, x, out, workspace,
                         static_cast<hipStream_t>(stream)),
          "moe launch");
  return SH_OK;
}

int sh_moe_layer_workspace_bytes(uint32_t n_tok, uint32_t top_k, uint64_t n_expert, uint64_t n_embd,
                                 uint64_t n_ff, uint64_t n_ff_shexp, const uint32_t* quants, uint64_t* bytes) {
  if (!quants || !bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const sh::MoeLayerTypes q{quants[0], quants[1], quants[2], quants[3], quants[4], quants[5], quants[6], quants[7]};
  // enough for either orientation of the stacks (whichever the shape allows)
  sh::MoeLayerPlan in_major, out_major;
  const bool a = n_tok > 0 && top_k > 0 && n_expert <= uint64_t(sh::kMoeMaxExperts) && n_embd <= (1u << 20) &&
                 n_ff <= (1u << 20) && n_ff_shexp <= (1u << 20) && q.up == q.gate &&
                 sh::moe_layer_plan(int(std::min<uint32_t>(n_tok, 1u << 30)), int(std::min<uint32_t>(top_k, 1u << 30)),
                                    int(n_expert), int(n_embd), int(n_ff), int(n_ff_shexp), q, &out_major, true);
  int rc = moe_layer_check(n_expert, n_embd, n_ff, n_ff_shexp, n_tok, top_k, q, &in_major);
  if (rc && !a) return rc;
  *bytes = std::max<uint64_t>(rc ? 0 : in_major.bytes, a ? out_major.bytes : 0);
  return SH_OK;
}

int sh_moe_layer_dev(const sh_expert_dev* t, uint64_t n_expert, uint64_t n_embd, uint64_t n_ff,
                     uint64_t n_ff_shexp, uint32_t n_tok, uint32_t top_k, const float* x, float* out,
                     void* workspace, uint64_t workspace_bytes, void* stream) {
  if (!t || !x || !out || !workspace) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const int om = orientation(t[1].flags, t[2].flags, t[3].flags);
  if (om < 0) return mixed_orientation();
  for (int i = 0; i < 8; ++i) {
    if (!t[i].data) return fail(SH_ERR_INVALID_ARGUMENT, "null tensor %d", i);
    if ((reinterpret_cast<uintptr_t>(t[i].data) & 1u) ||
        ((t[i].quant == SH_QUANT_Q8_0 || t[i].quant == SH_QUANT_F32 || t[i].quant == SH_QUANT_IQ4_XS) &&
         (reinterpret_cast<uintptr_t>(t[i].data) & 3u)))
      return fail(SH_ERR_INVALID_ARGUMENT, "misaligned tensor %d", i);
  }
  if (reinterpret_cast<uintptr_t>(x) & 15u) return fail(SH_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
  const sh::MoeLayerTypes q{t[0].quant, t[1].quant, t[2].quant, t[3].quant,
                            t[4].quant, t[5].quant, t[6].quant, t[7].quant};
  int rc;
  // gate / up [gr][gc] and down [gc][gr] per expert, by orientation
  const uint64_t gr = om ? n_ff : n_embd, gc = om ? n_embd : n_ff;
  const uint64_t dims[8][2] = {{n_expert, n_embd}, {gr, gc}, {gr, gc}, {gc, gr},
                               {n_ff_shexp, n_embd}, {n_ff_shexp, n_embd}, {n_embd, n_ff_shexp}, {1, n_embd}};
  for (int i = 0; i < 8; ++i)
    if ((rc = check_matrix(t[i].quant, dims[i][0], dims[i][1], 1, ~uint64_t(0), i == 0 || i >= 4))) return rc;
  sh::MoeLayerPlan plan;
  if ((rc = moe_layer_check(n_expert, n_embd, n_ff, n_ff_shexp, n_tok, top_k, q, &plan, om == 1))) return rc;
  if (workspace_bytes < plan.bytes)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace of %llu bytes, %llu needed",
                (unsigned long long)workspace_bytes, (unsigned long long)plan.bytes);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  auto q6 = [](const sh_expert_dev& d) { return reading(d.quant, d.flags); };
  const sh::MoeLayerTensors w{t[0].data, t[1].data, t[2].data, t[3].data, t[4].data, t[5].data, t[6].data,
                              t[7].data, q6(t[0]), q6(t[1]), q6(t[2]), q6(t[3]),
                              q6(t[4]), q6(t[5]), q6(t[6]), q6(t[7])};
  HIP_TRY(sh::launch_moe_layer(plan, q, w, x, out, workspace, static_cast<hipStream_t>(stream)),
          "moe layer launch");
  return SH_OK;
}

}  // extern "C"

int sh_matmul_workspace_bytes(uint32_t quant, uint64_t rows, uint64_t cols, uint32_t m, uint32_t mode,
                              uint64_t* bytes) {
  if (!bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null bytes");
  int rc = matmul_check(quant, rows, cols, m, mode);
  if (rc) return rc;
  *bytes = sh::matmul_workspace_bytes(int64_t(cols), int64_t(m), mode);
  return SH_OK;
}

int sh_matmul_dev(uint32_t quant, uint32_t flags, const void* w, uint64_t rows, uint64_t cols,
                  const float* x, uint32_t m, float* y, uint32_t mode, void* workspace,
                  uint64_t workspace_bytes, void* stream) {
  if (!w || !x || !y || !workspace) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  int rc = matmul_check(quant, rows, cols, m, mode);
  if (rc) return rc;
  const uint64_t need = sh::matmul_workspace_bytes(int64_t(cols), int64_t(m), mode);
  if (workspace_bytes < need)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace of %llu bytes, %llu needed",
                (unsigned long long)workspace_bytes, (unsigned long long)need);
  if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(x) & 15u) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned pointer (w needs 4 bytes, x 16, workspace 256)");
  HIP_TRY(sh::launch_matmul(quant, w, int64_t(rows), int64_t(cols), x, int64_t(m), y, mode, workspace,
                            reading(quant, flags), static_cast<hipStream_t>(stream)),
          "matmul launch");
  return SH_OK;
}

int sh_quantize_q8_dev(const float* x, uint64_t n, int8_t* codes, float* scales, float* code_sums,
                       void* stream) {
  if (!x || !codes || !scales || !code_sums) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if (n == 0 || n % 32 != 0 || n > (uint64_t(1) << 40))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "quantize: %llu values (a positive multiple of 32 needed)",
                (unsigned long long)n);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(codes) & 15u))
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned pointer (x and codes need 16 bytes)");
  HIP_TRY(sh::launch_quantize_q8(x, int64_t(n), codes, scales, code_sums, static_cast<hipStream_t>(stream)),
          "quantize launch");
  return SH_OK;
}

int sh_quantize_q8k_dev(const float* x, uint64_t n, int8_t* codes, float* scales, int32_t* sub_sums,
                        void* stream) {
  if (!x || !codes || !scales || !sub_sums) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if (n == 0 || n % 256 != 0 || n > (uint64_t(1) << 40))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "quantize: %llu values (a positive multiple of 256 needed)",
                (unsigned long long)n);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(codes) & 3u) ||
      (reinterpret_cast<uintptr_t>(scales) & 3u) || (reinterpret_cast<uintptr_t>(sub_sums) & 3u))
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned pointer (x needs 16 bytes, the outputs 4)");
  HIP_TRY(sh::launch_quantize_q8k(x, int64_t(n), codes, scales, sub_sums, static_cast<hipStream_t>(stream)),
          "quantize launch");
  return SH_OK;
}

// ---- the trait's elementwise methods ----------------------------------------

namespace {

int rowops_check(uint64_t rows, uint64_t n) {
  if (!sh::rowops_shape_ok(int64_t(rows > (uint64_t(1) << 62) ? (uint64_t(1) << 62) : rows),
                           int64_t(n > (uint64_t(1) << 62) ? (uint64_t(1) << 62) : n)))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "%llu rows of %llu floats is beyond the kernels' grids",
                (unsigned long long)rows, (unsigned long long)n);
  return SH_OK;
}

// Uploads `n` floats of each of up to two host slices into the context's
// input buffer (16-byte aligned pieces), runs `launch` on the device
// pointers, and copies the first piece back into `back`.
template <class F>
int run_rows(sh_context* c, const float* a, uint64_t na, const float* b, uint64_t nb, float* back,
             const char* what, F launch) {
  Guard gd(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  const size_t ab = sizeof(float) * na, bb = sizeof(float) * nb;
  const size_t a_al = (ab + 255) & ~size_t(255);
  int rc;
  if ((rc = c->d_in.ensure(a_al + bb, "input buffer")) || (rc = c->h_in.ensure(a_al + bb, "input staging")) ||
      (rc = c->h_out.ensure(ab, "output staging")))
    return rc;
  uint8_t* hi = static_cast<uint8_t*>(c->h_in.p);
  memcpy(hi, a, ab);
  if (nb) memcpy(hi + a_al, b, bb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, a_al + bb, c->stream), "upload");
  float* da = static_cast<float*>(c->d_in.p);
  const float* db = reinterpret_cast<const float*>(static_cast<uint8_t*>(c->d_in.p) + a_al);
  HIP_TRY(launch(da, db, c->stream), what);
  HIP_TRY(sh::launch_copy_bytes(c->d_in.p, c->h_out.dev, ab, c->stream), "readback");
  HIP_TRY(hipStreamSynchronize(c->stream), what);
  memcpy(back, c->h_out.p, ab);
  return SH_OK;
}

}  // namespace

int sh_rms_norm(sh_context* c, float* x, const float* w, uint64_t n, double eps) {
  if (!c || (n && (!x || !w))) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = rowops_check(1, n);
  if (rc || n == 0) return rc;
  return run_rows(c, x, n, w, n, x, "rms_norm", [&](float* dx, const float* dw, hipStream_t s) {
    return sh::launch_rms_norm(dx, dw, dx, 1, int64_t(n), eps, s);
  });
}

int sh_rope_neox(sh_context* c, float* head, uint64_t n, const sh_rope_cfg* cfg) {
  if (!c || !cfg || (n && !head)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = rowops_check(1, n);
  if (rc) return rc;
  // r = min(n_rot, head_dim, n) & ~1 (ops.rs:123): the slice length bounds
  // the rotated span, so the kernel's head_dim is n here
  const uint64_t r = std::min(std::min(cfg->n_rot, cfg->head_dim), n) & ~uint64_t(1);
  if (r == 0) return SH_OK;
  return run_rows(c, head, n, nullptr, 0, head, "rope_neox", [&](float* dx, const float*, hipStream_t s) {
    return sh::launch_rope_neox(dx, 1, int64_t(n), int64_t(r), cfg->pos, 1, cfg->freq_base, s);
  });
}

int sh_softmax(sh_context* c, float* xs, uint64_t n) {
  if (!c || (n && !xs)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = rowops_check(1, n);
  if (rc || n == 0) return rc;
  return run_rows(c, xs, n, nullptr, 0, xs, "softmax", [&](float* dx, const float*, hipStream_t s) {
    return sh::launch_softmax(dx, 1, int64_t(n), s);
  });
}

int sh_l2_norm(sh_context* c, float* head, uint64_t n, double eps) {
  if (!c || (n && !head)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = rowops_check(1, n);
  if (rc || n == 0) return rc;
  return run_rows(c, head, n, nullptr, 0, head, "l2_norm", [&](float* dx, const float*, hipStream_t s) {
    return sh::launch_l2_norm(dx, 1, int64_t(n), eps, s);
  });
}

int sh_add(sh_context* c, float* a, const float* b, uint64_t n) {
  if (!c || (n && (!a || !b))) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = rowops_check(1, n);
  if (rc || n == 0) return rc;
  return run_rows(c, a, n, b, n, a, "add", [&](float* da, const float* db, hipStream_t s) {
    return sh::launch_add(da, db, int64_t(n), s);
  });
}

int sh_rms_norm_dev(const float* x, const float* w, float* out, uint64_t rows, uint64_t n, double eps,
                    void* stream) {
  int rc = rowops_check(rows, n);
  if (rc || rows == 0 || n == 0) return rc;
  if (!x || !w || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  HIP_TRY(sh::launch_rms_norm(x, w, out, int64_t(rows), int64_t(n), eps, static_cast<hipStream_t>(stream)),
          "rms_norm launch");
  return SH_OK;
}

int sh_l2_norm_dev(float* x, uint64_t rows, uint64_t n, double eps, void* stream) {
  int rc = rowops_check(rows, n);
  if (rc || rows == 0 || n == 0) return rc;
  if (!x) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  HIP_TRY(sh::launch_l2_norm(x, int64_t(rows), int64_t(n), eps, static_cast<hipStream_t>(stream)),
          "l2_norm launch");
  return SH_OK;
}

int sh_softmax_dev(float* x, uint64_t rows, uint64_t n, void* stream) {
  int rc = rowops_check(rows, n);
  if (rc || rows == 0 || n == 0) return rc;
  if (!x) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  HIP_TRY(sh::launch_softmax(x, int64_t(rows), int64_t(n), static_cast<hipStream_t>(stream)), "softmax launch");
  return SH_OK;
}

int sh_rope_neox_dev(float* x, uint64_t rows, uint64_t heads_per_pos, const sh_rope_cfg* cfg, void* stream) {
  if (!cfg) return fail(SH_ERR_INVALID_ARGUMENT, "null cfg");
  if (heads_per_pos == 0) return fail(SH_ERR_INVALID_ARGUMENT, "heads_per_pos is 0");
  int rc = rowops_check(rows, cfg->head_dim);
  if (rc) return rc;
  const uint64_t r = std::min(cfg->n_rot, cfg->head_dim) & ~uint64_t(1);
  if (rows == 0 || r == 0) return SH_OK;
  if (!x) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  if (rows * (r / 2) / 256 >= (uint64_t(1) << 31) || heads_per_pos > (uint64_t(1) << 62))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "rope over %llu heads is beyond the kernel's grid",
                (unsigned long long)rows);
  HIP_TRY(sh::launch_rope_neox(x, int64_t(rows), int64_t(cfg->head_dim), int64_t(r), cfg->pos,
                               int64_t(heads_per_pos), cfg->freq_base, static_cast<hipStream_t>(stream)),
          "rope launch");
  return SH_OK;
}

int sh_add_dev(float* a, const float* b, uint64_t n, void* stream) {
  int rc = rowops_check(1, n);
  if (rc || n == 0) return rc;
  if (!a || !b) return fail(SH_ERR_INVALID_ARGUMENT, "null pointer");
  HIP_TRY(sh::launch_add(a, b, int64_t(n), static_cast<hipStream_t>(stream)), "add launch");
  return SH_OK;
}

// ---- GGUF weight source ---------------------------------------------------

struct sh_gguf {
  sh::GgufFile* f;
  bool owned;  // false for a shard handle lent out by a model
};

struct sh_gguf_model {
  sh::GgufModel* m;
  std::vector<sh_gguf> shards;  // borrowed handles onto m's files
};

namespace {

int gguf_fail(sh::GgufErr e, const std::string& msg) {
  switch (e) {
    case sh::GgufErr::kOk: return SH_OK;
    case sh::GgufErr::kIo: return fail(SH_ERR_IO, "%s", msg.c_str());
    case sh::GgufErr::kTruncated: return fail(SH_ERR_TRUNCATED, "%s", msg.c_str());
    case sh::GgufErr::kUnsupportedQuant: return fail(SH_ERR_UNSUPPORTED_QUANT, "%s", msg.c_str());
    default: return fail(SH_ERR_FORMAT, "%s", msg.c_str());
  }
}

const sh::GgufMeta* meta_of(const sh_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->f->meta.find(key);
  return it == g->f->meta.end() ? nullptr : &it->second;
}

bool meta_integer(uint32_t t) { return t <= 5 || t == 7 || t == 10 || t == 11; }  // MetaValue::as_int
bool meta_number(uint32_t t) { return t != 8 && t != 9; }                          // MetaValue::is_num

}  // namespace

int sh_gguf_open(const char* path, sh_gguf** out) {
  if (!path || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  sh::GgufFile* f = nullptr;
  std::string msg;
  const sh::GgufErr e = sh::gguf_open(path, &f, &msg);
  if (e != sh::GgufErr::kOk) return gguf_fail(e, msg);
  *out = new sh_gguf{f, true};
  return SH_OK;
}

int sh_gguf_close(sh_gguf* g) {
  if (g && g->owned) {
    delete g->f;
    delete g;
  }
  return SH_OK;
}

int sh_gguf_model_open(const char* any_shard, sh_gguf_model** out) {
  if (!any_shard || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  sh::GgufModel* m = nullptr;
  std::string msg;
  const sh::GgufErr e = sh::gguf_model_open(any_shard, &m, &msg);
  if (e != sh::GgufErr::kOk) return gguf_fail(e, msg);
  sh_gguf_model* h = new sh_gguf_model{m, {}};
  for (sh::GgufFile* f : m->shards) h->shards.push_back(sh_gguf{f, false});
  *out = h;
  return SH_OK;
}

int sh_gguf_model_close(sh_gguf_model* m) {
  if (m) {
    delete m->m;
    delete m;
  }
  return SH_OK;
}

int sh_gguf_model_shards(const sh_gguf_model* m, uint64_t* n) {
  if (!m || !n) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  *n = m->shards.size();
  return SH_OK;
}

int sh_gguf_model_shard(sh_gguf_model* m, uint64_t i, sh_gguf** shard) {
  if (!m || !shard) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (i >= m->shards.size()) return fail(SH_ERR_NOT_FOUND, "shard %llu of %zu", (unsigned long long)i, m->shards.size());
  *shard = &m->shards[i];
  return SH_OK;
}

int sh_gguf_model_find(const sh_gguf_model* m, const char* name, uint64_t* shard, uint64_t* index) {
  if (!m || !name || !shard || !index) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  auto it = m->m->index.find(name);
  if (it == m->m->index.end()) return fail(SH_ERR_NOT_FOUND, "no tensor named %s", name);
  *shard = it->second.first;
  *index = it->second.second;
  return SH_OK;
}

int sh_gguf_header(const sh_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv, uint64_t* alignment,
                   uint64_t* data_start, uint64_t* file_size) {
  if (!g) return fail(SH_ERR_INVALID_ARGUMENT, "null file");
  if (version) *version = g->f->version;
  if (n_tensors) *n_tensors = g->f->tensors.size();
  if (n_kv) *n_kv = g->f->n_kv;
  if (alignment) *alignment = g->f->alignment;
  if (data_start) *data_start = g->f->data_start;
  if (file_size) *file_size = g->f->size;
  return SH_OK;
}

int sh_gguf_tensor(const sh_gguf* g, uint64_t index, sh_gguf_tensor_info* out) {
  if (!g || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (index >= g->f->tensors.size())
    return fail(SH_ERR_NOT_FOUND, "tensor %llu of %llu", (unsigned long long)index,
                (unsigned long long)g->f->tensors.size());
  const sh::GgufTensor& t = g->f->tensors[index];
  out->name = t.name.c_str();
  out->n_dims = uint32_t(t.shape.size());
  out->type = t.ty;
  for (int d = 0; d < 4; ++d) out->shape[d] = d < int(t.shape.size()) ? t.shape[d] : 1;
  out->offset = t.offset;
  std::string msg;
  uint64_t nb = 0;
  out->nbytes = sh::gguf_payload_bytes(t, &nb, &msg) == sh::GgufErr::kOk ? nb : 0;
  return SH_OK;
}

int sh_gguf_find(const sh_gguf* g, const char* name, uint64_t* index) {
  if (!g || !name || !index) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  auto it = g->f->index.find(name);
  if (it == g->f->index.end()) return fail(SH_ERR_NOT_FOUND, "no tensor named %s", name);
  *index = it->second;
  return SH_OK;
}

int sh_gguf_tensor_data(const sh_gguf* g, uint64_t index, const uint8_t** data, uint64_t* nbytes) {
  if (!g || !data || !nbytes) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (index >= g->f->tensors.size()) return fail(SH_ERR_NOT_FOUND, "tensor %llu", (unsigned long long)index);
  std::string msg;
  return gguf_fail(sh::gguf_tensor_data(*g->f, g->f->tensors[index], data, nbytes, &msg), msg);
}

int sh_gguf_meta_type(const sh_gguf* g, const char* key, uint32_t* type, uint32_t* elem, uint64_t* count) {
  const sh::GgufMeta* m = meta_of(g, key);
  if (!m) return fail(SH_ERR_NOT_FOUND, "no metadata key %s", key ? key : "(null)");
  if (type) *type = m->ty;
  if (elem) *elem = m->elem;
  if (count) *count = m->count;
  return SH_OK;
}

int sh_gguf_meta_int(const sh_gguf* g, const char* key, int64_t* value) {
  const sh::GgufMeta* m = meta_of(g, key);
  if (!m || !value || !meta_integer(m->ty))
    return fail(SH_ERR_NOT_FOUND, "no integer metadata key %s", key ? key : "(null)");
  *value = m->i;
  return SH_OK;
}

int sh_gguf_meta_float(const sh_gguf* g, const char* key, double* value) {
  const sh::GgufMeta* m = meta_of(g, key);
  if (!m || !value || !meta_number(m->ty))
    return fail(SH_ERR_NOT_FOUND, "no numeric metadata key %s", key ? key : "(null)");
  *value = (m->ty == 6 || m->ty == 12) ? m->f : double(m->i);
  return SH_OK;
}

int sh_gguf_meta_str(const sh_gguf* g, const char* key, const char** s, uint64_t* len) {
  const sh::GgufMeta* m = meta_of(g, key);
  if (!m || !s || m->ty != 8) return fail(SH_ERR_NOT_FOUND, "no string metadata key %s", key ? key : "(null)");
  *s = m->s.c_str();
  if (len) *len = m->s.size();
  return SH_OK;
}

int sh_upload_gguf_tensor(sh_context* c, const sh_gguf* g, uint64_t index, uint64_t key) {
  if (!c || !g) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (index >= g->f->tensors.size()) return fail(SH_ERR_NOT_FOUND, "tensor %llu", (unsigned long long)index);
  const sh::GgufTensor& t = g->f->tensors[index];
  if (!sh::gemv_quant(t.ty) && !sh::plain_quant(t.ty))
    return fail(SH_ERR_UNSUPPORTED_QUANT, "%s: type %u has no device kernel here", t.name.c_str(), t.ty);
  if (t.shape.size() > 3)
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "%s: %zu dims (matrices and expert stacks only)", t.name.c_str(),
                t.shape.size());
  const uint8_t* data = nullptr;
  uint64_t nb = 0;
  std::string msg;
  const sh::GgufErr e = sh::gguf_tensor_data(*g->f, t, &data, &nb, &msg);
  if (e != sh::GgufErr::kOk) return gguf_fail(e, msg);
  // GGUF dims, fastest first: [cols, rows, n_expert] (weights.rs:14-34)
  const uint64_t cols = t.shape[0];
  const uint64_t rows = t.shape.size() > 1 ? t.shape[1] : 1;
  const uint64_t n_expert = t.shape.size() > 2 ? t.shape[2] : 1;
  if (cols % uint64_t(sh::geometry(t.ty).block) != 0)
    return fail(SH_ERR_TRUNCATED, "%s: %llu columns are not whole blocks", t.name.c_str(), (unsigned long long)cols);
  Guard gd(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident* r = nullptr;
  return resident(c, key, t.ty, n_expert, rows, cols, data, nb, &r);
}

int sh_weight_upload(sh_context* c, uint64_t key, uint32_t quant, uint64_t n_expert, uint64_t rows, uint64_t cols,
                     const uint8_t* data, uint64_t src_row_pitch) {
  if (!c || !data) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  if (!sh::gemv_quant(quant) && !sh::plain_quant(quant))
    return fail(SH_ERR_UNSUPPORTED_QUANT, "quant type id %u has no device kernel here", quant);
  const sh::Geometry g = sh::geometry(quant);
  if (cols % uint64_t(g.block) != 0)
    return fail(SH_ERR_TRUNCATED, "cols %llu is not a whole number of blocks", (unsigned long long)cols);
  const uint64_t rb = cols / uint64_t(g.block) * uint64_t(g.bytes);
  const uint64_t n_rows = n_expert * rows;
  if (n_expert == 0 || (rows && n_rows / rows != n_expert) || (rb && n_rows > ~uint64_t(0) / rb))
    return fail(SH_ERR_INVALID_ARGUMENT, "bad tensor shape");
  if (src_row_pitch != 0 && src_row_pitch < rb)
    return fail(SH_ERR_INVALID_ARGUMENT, "row pitch %llu is below the row size %llu",
                (unsigned long long)src_row_pitch, (unsigned long long)rb);
  Guard gd(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  Resident* r = nullptr;
  if (src_row_pitch == 0 || src_row_pitch == rb || n_rows <= 1)
    return resident(c, key, quant, n_expert, rows, cols, data, n_rows * rb, &r);
  // pitched rows: packed into a host copy first
  std::vector<uint8_t> packed;
  try {
    packed.resize(size_t(n_rows * rb));
  } catch (const std::bad_alloc&) {
    return fail(SH_ERR_OUT_OF_MEMORY, "host memory for re-pitching %llu rows", (unsigned long long)n_rows);
  }
  for (uint64_t i = 0; i < n_rows; ++i) memcpy(packed.data() + i * rb, data + i * src_row_pitch, size_t(rb));
  return resident(c, key, quant, n_expert, rows, cols, packed.data(), n_rows * rb, &r);
}

int sh_ffn_workspace_bytes(uint32_t n_tok, uint64_t n_embd, uint64_t n_ff, uint64_t* bytes) {
  if (!bytes) return fail(SH_ERR_INVALID_ARGUMENT, "null bytes");
  if (n_tok == 0 || n_embd == 0 || n_ff == 0 || n_embd > (uint64_t(1) << 20) || n_ff > (uint64_t(1) << 20))
    return fail(SH_ERR_UNSUPPORTED_SHAPE, "ffn shape");
  *bytes = sh::ffn_workspace_bytes(n_tok, int64_t(n_embd), int64_t(n_ff));
  return SH_OK;
}

// Validation shared by sh_ffn_dev and sh_ffn_dev_noalloc (everything but
// the workspace, which each checks itself).
static int ffn_dev_check(const sh_expert_dev* t, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok, const float* x,
                         const float* post_norm, const float* out, uint64_t* need) {
  if (!t || !x || !post_norm || !out) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  int rc = sh_ffn_workspace_bytes(n_tok, n_embd, n_ff, need);
  if (rc) return rc;
  const uint64_t dims[3][2] = {{n_ff, n_embd}, {n_ff, n_embd}, {n_embd, n_ff}};
  for (int i = 0; i < 3; ++i) {
    if (!t[i].data) return fail(SH_ERR_INVALID_ARGUMENT, "null tensor %d", i);
    if ((rc = check_matrix(t[i].quant, dims[i][0], dims[i][1], 1, ~uint64_t(0), true))) return rc;
    if (!sh::gemv_shape_ok(t[i].quant, int64_t(dims[i][0]), int64_t(dims[i][1]), 1))
      return fail(SH_ERR_UNSUPPORTED_SHAPE, "ffn tensor %d: %llux%llu of type %u", i,
                  (unsigned long long)dims[i][0], (unsigned long long)dims[i][1], t[i].quant);
    if ((reinterpret_cast<uintptr_t>(t[i].data) & 1u) ||
        ((t[i].quant == SH_QUANT_Q8_0 || t[i].quant == SH_QUANT_F32 || t[i].quant == SH_QUANT_IQ4_XS) &&
         (reinterpret_cast<uintptr_t>(t[i].data) & 3u)))
      return fail(SH_ERR_INVALID_ARGUMENT, "misaligned tensor %d", i);
  }
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u) || n_embd % 4 != 0 ||
      n_ff % 4 != 0)
    return fail(SH_ERR_INVALID_ARGUMENT, "misaligned x or out (or n_embd, n_ff not multiples of 4)");
  return SH_OK;
}

static hipError_t ffn_dev_launch(const sh_expert_dev* t, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok,
                                 const float* x, const float* post_norm, double eps, float* out, void* workspace,
                                 void* stream) {
  auto q6 = [](const sh_expert_dev& d) { return reading(d.quant, d.flags); };
  return sh::launch_ffn(t[0].quant, t[1].quant, t[2].quant, t[0].data, t[1].data, t[2].data, q6(t[0]),
                        q6(t[1]), q6(t[2]), int64_t(n_embd), int64_t(n_ff), int(n_tok), x, post_norm, eps,
                        out, workspace, static_cast<hipStream_t>(stream));
}

int sh_ffn_dev(const sh_expert_dev* t, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok, const float* x,
               const float* post_norm, double eps, float* out, void* workspace, uint64_t workspace_bytes,
               void* stream) {
  uint64_t need = 0;
  int rc = ffn_dev_check(t, n_embd, n_ff, n_tok, x, post_norm, out, &need);
  if (rc) return rc;
  if (!workspace) return fail(SH_ERR_INVALID_ARGUMENT, "null workspace");
  if (workspace_bytes < need)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace of %llu bytes, %llu needed", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(SH_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  HIP_TRY(ffn_dev_launch(t, n_embd, n_ff, n_tok, x, post_norm, eps, out, workspace, stream), "ffn launch");
  return SH_OK;
}

// The current device's address of `scratch`, looked up once per device (with
// that device current) and kept.
static int scratch_address(void** out) {
  static_assert(sizeof(scratch) == kScratchBytes, "scratch size");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices) return fail(SH_ERR_NO_DEVICE, "device %d: no scratch slot", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail(SH_ERR_DEVICE, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SH_OK;
}

int sh_ffn_dev_noalloc(const sh_expert_dev* t, uint64_t n_embd, uint64_t n_ff, uint32_t n_tok, const float* x,
                       const float* post_norm, double eps, float* out, void* stream) {
  uint64_t need = 0;
  int rc = ffn_dev_check(t, n_embd, n_ff, n_tok, x, post_norm, out, &need);
  if (rc) return rc;
  if (need > kScratchBytes)
    return fail(SH_ERR_UNSUPPORTED_SHAPE,
                "ffn of %u tokens at %llu x %llu needs %llu bytes of scratch; the allocation-free path has %llu",
                n_tok, (unsigned long long)n_embd, (unsigned long long)n_ff, (unsigned long long)need,
                (unsigned long long)kScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  HIP_TRY(ffn_dev_launch(t, n_embd, n_ff, n_tok, x, post_norm, eps, out, ws, stream), "ffn launch");
  return SH_OK;
}

int sh_ffn(sh_context* c, const sh_quant_tensor* gate, const sh_quant_tensor* up, const sh_quant_tensor* down,
           const float* post_norm, double eps, uint32_t n_tok, float* x) {
  if (!c || !gate || !up || !down || !post_norm || (!x && n_tok)) return fail(SH_ERR_INVALID_ARGUMENT, "null argument");
  const uint64_t n_embd = gate->cols, n_ff = gate->rows;
  if (up->rows != n_ff || up->cols != n_embd || down->rows != n_embd || down->cols != n_ff)
    return fail(SH_ERR_SHAPE, "ffn: gate/up must be [n_ff][n_embd] and down [n_embd][n_ff]");
  const sh_quant_tensor* t[3] = {gate, up, down};
  int rc;
  for (int i = 0; i < 3; ++i)
    if ((rc = check_matrix(t[i]->quant, t[i]->rows, t[i]->cols, 1, t[i]->nbytes, true))) return rc;
  if (n_tok == 0 || n_embd == 0 || n_ff == 0) return SH_OK;
  uint64_t need = 0;
  if ((rc = sh_ffn_workspace_bytes(n_tok, n_embd, n_ff, &need))) return rc;
  for (int i = 0; i < 3; ++i)
    if (!sh::gemv_shape_ok(t[i]->quant, int64_t(t[i]->rows), int64_t(t[i]->cols), 1))
      return fail(SH_ERR_UNSUPPORTED_SHAPE, "ffn tensor %d: %llux%llu of type %u", i,
                  (unsigned long long)t[i]->rows, (unsigned long long)t[i]->cols, t[i]->quant);
  if (n_embd % 4 != 0 || n_ff % 4 != 0) return fail(SH_ERR_UNSUPPORTED_SHAPE, "n_embd and n_ff must be multiples of 4");
  Guard g(c);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  // the three matrices resident at once (pinned to this call)
  void* dev[3] = {};
  for (int i = 0; i < 3; ++i) {
    Resident* r = nullptr;
    const uint64_t nb = t[i]->rows * uint64_t(sh::byte_size(t[i]->quant, int64_t(t[i]->cols)));
    if ((rc = resident(c, t[i]->key, t[i]->quant, 1, t[i]->rows, t[i]->cols, t[i]->data, nb, &r))) return rc;
    dev[i] = r->dev;
  }
  // x and post_norm in one upload (post_norm 256-byte aligned after x)
  const size_t xb = sizeof(float) * n_tok * n_embd, nb = sizeof(float) * n_embd;
  const size_t x_al = (xb + 255) & ~size_t(255);
  if ((rc = c->d_in.ensure(x_al + nb, "x buffer")) || (rc = c->d_blk.ensure(need, "workspace")) ||
      (rc = c->h_in.ensure(x_al + nb, "x staging")) || (rc = c->h_out.ensure(xb, "out staging")))
    return rc;
  uint8_t* hi = static_cast<uint8_t*>(c->h_in.p);
  memcpy(hi, x, xb);
  memcpy(hi + x_al, post_norm, nb);
  HIP_TRY(sh::launch_copy_bytes(c->h_in.dev, c->d_in.p, x_al + nb, c->stream), "x upload");
  float* dx = static_cast<float*>(c->d_in.p);
  const float* dn = reinterpret_cast<const float*>(static_cast<uint8_t*>(c->d_in.p) + x_al);
  HIP_TRY(sh::launch_ffn(gate->quant, up->quant, down->quant, dev[0], dev[1], dev[2],
                         reading(gate->quant, gate->flags), reading(up->quant, up->flags),
                         reading(down->quant, down->flags), int64_t(n_embd), int64_t(n_ff), int(n_tok), dx, dn, eps, dx, c->d_blk.p,
                         c->stream),
          "ffn launch");
  HIP_TRY(sh::launch_copy_bytes(dx, c->h_out.dev, xb, c->stream), "x readback");
  HIP_TRY(hipStreamSynchronize(c->stream), "ffn");
  memcpy(x, c->h_out.p, xb);
  return SH_OK;
}
