// Host side of the C ABI declared in include/qmm.h.
//
// Plain C++ over the HIP runtime: device memory with hipMalloc/hipMemcpyAsync,
// kernels from the embedded gfx950 code object through hipModuleLoadData /
// hipModuleGetFunction / hipModuleLaunchKernel. No torch types cross this
// boundary; callers pass raw device pointers and a hipStream_t.
#include "qmm.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

extern "C" const unsigned char qmm_code_object_start[];
extern "C" const unsigned char qmm_code_object_end[];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace

// Error reporting for the library's other translation units (qmm_gguf.cpp).
__attribute__((visibility("hidden"))) int qmm_internal_fail(int code, const char* msg) { return fail(code, "%s", msg); }

namespace {

#define QMM_HIP(expr)                                                                 \
  do {                                                                                \
    hipError_t e_ = (expr);                                                           \
    if (e_ != hipSuccess) return fail(QMM_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define QMM_TRY(expr)          \
  do {                         \
    int rc_ = (expr);          \
    if (rc_ != QMM_OK) return rc_; \
  } while (0)

enum { kFmtQ80 = 0, kFmtQ4K = 1, kFmtQ6K = 2 };

int fmt_of(int dtype) {
  switch (dtype) {
    case QMM_Q8_0: return kFmtQ80;
    case QMM_Q4K: return kFmtQ4K;
    case QMM_Q6K: return kFmtQ6K;
    default: return -1;
  }
}

const char* fmt_name(int fmt) { return fmt == kFmtQ80 ? "q8_0" : fmt == kFmtQ4K ? "q4k" : "q6k"; }

// Kernel handles of one device: an insert-only open-addressing table read
// without a lock (a launch hashes its name and probes; only a miss, the first
// launch of a kernel on the device, takes the mutex and asks the runtime).
struct KernelEntry {
  uint64_t hash;
  std::string name;
  hipFunction_t fn;
};
constexpr int kKernelSlots = 8192;  // > 4x the kernels of the code object

struct Device {
  hipModule_t module = nullptr;
  std::atomic<const KernelEntry*> slots[kKernelSlots];
  int max_lds = 0;
  int num_cu = 0;
  Device() {
    for (auto& e : slots) e.store(nullptr, std::memory_order_relaxed);
  }
};

std::mutex g_mu;
std::atomic<Device*> g_dev[64] = {};

// Launch-shape and kernel-choice overrides for tuning sweeps and tests: the
// QMM_* variables below are read into a snapshot at the first launch and again
// at every qmm_reload_tuning(), never per launch.
//   QMM_GEMV_CFG="W,R,U" (waves per workgroup, rows per wave, load iterations
//   per batch), QMM_GEMV_WAVES_PER_CU (resident waves the grid is sized for),
//   QMM_GEMV1=0 (the general kernel for one activation row too), QMM_GEMV1P=<P>
//   (the prefetch ring's depth; 0 never), and the GEMM / MoE choices named
//   where they are used.
enum EnvKey {
  kEnvGemv1, kEnvGemv1p, kEnvGemvCfg, kEnvGemvWavesPerCu, kEnvGemvRows, kEnvSplitK, kEnvMmq2, kEnvMmq,
  kEnvMmq4Bn, kEnvMmq1, kEnvMmqXcd, kEnvMoeGemv, kEnvMoeMmq, kEnvMoeBm, kEnvMoeSplitK, kEnvMoeGrouped, kEnvGroupedP,
  kEnvGroupedWgs, kEnvStreamK, kEnvGemvm, kEnvMmq6, kEnvMmq8, kEnvMoeTails, kEnvFfnPair, kEnvQkvSeparate, kEnvAttnOSeparate, kEnvCount
};
const char* const kEnvNames[kEnvCount] = {
    "QMM_GEMV1", "QMM_GEMV1P", "QMM_GEMV_CFG", "QMM_GEMV_WAVES_PER_CU", "QMM_GEMV_ROWS", "QMM_SPLITK",
    "QMM_MMQ2", "QMM_MMQ", "QMM_MMQ4_BN", "QMM_MMQ1", "QMM_MMQ_XCD", "QMM_MOE_GEMV", "QMM_MOE_MMQ",
    "QMM_MOE_BM", "QMM_MOE_SPLITK", "QMM_MOE_GROUPED", "QMM_GROUPED_P", "QMM_GROUPED_WGS",
    "QMM_STREAMK", "QMM_GEMVM", "QMM_MMQ6", "QMM_MMQ8", "QMM_MOE_TAILS", "QMM_FFN_SEPARATE", "QMM_QKV_SEPARATE",
    "QMM_ATTN_O_SEPARATE"};

struct Tuning {
  int w = 0, r = 0, u = 0, waves_per_cu = 0, gemv1 = 1, gemv1p = -1;
};

struct EnvSnapshot {
  bool set[kEnvCount];
  char val[kEnvCount][48];
  Tuning tu;
};

std::mutex g_env_mu;
std::atomic<const EnvSnapshot*> g_env{nullptr};

const EnvSnapshot* env_read() {
  EnvSnapshot* e = new EnvSnapshot();
  for (int k = 0; k < kEnvCount; ++k) {
    const char* v = getenv(kEnvNames[k]);
    e->set[k] = v != nullptr;
    snprintf(e->val[k], sizeof(e->val[k]), "%s", v ? v : "");
  }
  Tuning& t = e->tu;
  if (e->set[kEnvGemv1]) t.gemv1 = atoi(e->val[kEnvGemv1]);
  if (e->set[kEnvGemv1p]) t.gemv1p = atoi(e->val[kEnvGemv1p]);
  if (e->set[kEnvGemvCfg] && sscanf(e->val[kEnvGemvCfg], "%d,%d,%d", &t.w, &t.r, &t.u) != 3) t.w = t.r = t.u = 0;
  if (e->set[kEnvGemvWavesPerCu]) t.waves_per_cu = atoi(e->val[kEnvGemvWavesPerCu]);
  return e;
}

const EnvSnapshot* env_snapshot() {
  const EnvSnapshot* e = g_env.load(std::memory_order_acquire);
  if (e) return e;
  std::lock_guard<std::mutex> lk(g_env_mu);
  e = g_env.load(std::memory_order_acquire);
  if (!e) {
    e = env_read();
    g_env.store(e, std::memory_order_release);
  }
  return e;
}

// The override's value, or nullptr when it is not set.
const char* env(EnvKey k) {
  const EnvSnapshot* e = env_snapshot();
  return e->set[k] ? e->val[k] : nullptr;
}

const Tuning& tuning() { return env_snapshot()->tu; }

int current_device(Device** out) {
  int dev = 0;
  QMM_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(QMM_ERR_INVALID, "device ordinal %d out of range", dev);
  Device* have = g_dev[dev].load(std::memory_order_acquire);
  if (have) {
    *out = have;
    return QMM_OK;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_dev[dev].load(std::memory_order_acquire)) {
    Device* d = new Device();
    hipError_t e = hipModuleLoadData(&d->module, qmm_code_object_start);
    if (e != hipSuccess) {
      delete d;
      return fail(QMM_ERR_NO_KERNEL, "hipModuleLoadData(gfx950 code object) on device %d: %s", dev,
                  hipGetErrorString(e));
    }
    e = hipDeviceGetAttribute(&d->max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&d->num_cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) {
      (void)hipModuleUnload(d->module);
      delete d;
      return fail(QMM_ERR_HIP, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
    }
    g_dev[dev].store(d, std::memory_order_release);
  }
  *out = g_dev[dev].load(std::memory_order_acquire);
  return QMM_OK;
}

uint64_t name_hash(const char* s) {  // FNV-1a
  uint64_t h = 1469598103934665603ull;
  for (; *s; ++s) h = (h ^ (unsigned char)*s) * 1099511628211ull;
  return h;
}

int kernel(Device* d, const char* name, hipFunction_t* f) {
  const uint64_t h = name_hash(name);
  const unsigned start = (unsigned)(h % kKernelSlots);
  for (unsigned i = 0; i < kKernelSlots; ++i) {
    const KernelEntry* e = d->slots[(start + i) % kKernelSlots].load(std::memory_order_acquire);
    if (!e) break;
    if (e->hash == h && e->name == name) {
      *f = e->fn;
      return QMM_OK;
    }
  }
  std::lock_guard<std::mutex> lk(g_mu);
  unsigned i = 0;
  for (; i < kKernelSlots; ++i) {  // again under the lock: another thread may have added it
    const KernelEntry* e = d->slots[(start + i) % kKernelSlots].load(std::memory_order_acquire);
    if (!e) break;
    if (e->hash == h && e->name == name) {
      *f = e->fn;
      return QMM_OK;
    }
  }
  if (i == kKernelSlots) return fail(QMM_ERR_NO_KERNEL, "kernel table full looking up %s", name);
  hipFunction_t fn = nullptr;
  hipError_t err = hipModuleGetFunction(&fn, d->module, name);
  if (err != hipSuccess || !fn) {
    // The failed lookup also sets the runtime's last error; clear it so the
    // caller's next unrelated HIP call (e.g. a graph capture) does not report it.
    (void)hipGetLastError();
    return fail(QMM_ERR_NO_KERNEL, "kernel %s missing from the code object: %s", name, hipGetErrorString(err));
  }
  d->slots[(start + i) % kKernelSlots].store(new KernelEntry{h, name, fn}, std::memory_order_release);
  *f = fn;
  return QMM_OK;
}

int launch(Device* d, const char* name, unsigned grid, unsigned block, unsigned lds, hipStream_t s, void** args) {
  hipFunction_t f;
  QMM_TRY(kernel(d, name, &f));
  if (grid == 0) return QMM_OK;
  QMM_HIP(hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, lds, s, args, nullptr));
  return QMM_OK;
}

unsigned ceil_div(long long a, long long b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

struct qmm_qtensor {
  int dtype;
  int64_t n, k;
  int device;
  void* data;    // device layout (see qmm_common.h)
  size_t bytes;  // == GGML bytes of the tensor
};

extern "C" {

const char* qmm_last_error(void) { return g_err.c_str(); }

void qmm_reload_tuning(void) {
  const EnvSnapshot* e = env_read();
  std::lock_guard<std::mutex> lk(g_env_mu);
  // the previous snapshot stays allocated: a launch on another thread may still read it
  g_env.store(e, std::memory_order_release);
}

// qmm_noalloc.hip: resolves the allocation-free entry point's device scratch
// on the current device (set-up, once per device).
__attribute__((visibility("hidden"))) int qmm_internal_noalloc_setup(void** out);

int qmm_init(int device) {
  int prev = 0;
  QMM_HIP(hipGetDevice(&prev));
  QMM_HIP(hipSetDevice(device));
  Device* d;
  int rc = current_device(&d);
  if (rc == QMM_OK) rc = qmm_internal_noalloc_setup(nullptr);
  (void)hipSetDevice(prev);
  return rc;
}

int qmm_block_size(int dtype) {
  switch (dtype) {
    case QMM_Q8_0: return 32;
    case QMM_Q4K: case QMM_Q6K: case QMM_Q8K: return 256;
    default: return -1;
  }
}

int qmm_type_size(int dtype) {
  switch (dtype) {
    case QMM_Q8_0: return 34;
    case QMM_Q4K: return 144;
    case QMM_Q6K: return 210;
    case QMM_Q8K: return 292;
    default: return -1;
  }
}

int qmm_vec_dot_type(int dtype) {
  switch (dtype) {
    case QMM_Q8_0: return QMM_Q8_0;
    case QMM_Q4K: case QMM_Q6K: return QMM_Q8K;
    default: return -1;
  }
}

static int check_shape(int dtype, int64_t n, int64_t k) {
  if (fmt_of(dtype) < 0) return fail(QMM_ERR_INVALID, "unsupported weight dtype %d", dtype);
  const int bs = qmm_block_size(dtype);
  if (n <= 0 || k <= 0) return fail(QMM_ERR_INVALID, "empty shape (%lld, %lld)", (long long)n, (long long)k);
  if (k % bs) return fail(QMM_ERR_INVALID, "k = %lld is not a multiple of the block size %d", (long long)k, bs);
  if (n > (1LL << 31) - 1 || k > (1LL << 31) - 1) return fail(QMM_ERR_INVALID, "shape too large");
  return QMM_OK;
}

static int alloc_tensor(int dtype, int64_t n, int64_t k, qmm_qtensor** out) {
  qmm_qtensor* t = new qmm_qtensor();
  t->dtype = dtype;
  t->n = n;
  t->k = k;
  QMM_HIP(hipGetDevice(&t->device));
  t->bytes = (size_t)(n * (k / qmm_block_size(dtype))) * qmm_type_size(dtype);
  hipError_t e = hipMalloc(&t->data, t->bytes);
  if (e != hipSuccess) {
    delete t;
    return fail(QMM_ERR_OOM, "hipMalloc(%zu): %s", t->bytes, hipGetErrorString(e));
  }
  *out = t;
  return QMM_OK;
}

// Device GGML bytes -> the tensor's device layout.
static int ggml_to_dev(Device* d, qmm_qtensor* t, const void* src, hipStream_t s) {
  const int fmt = fmt_of(t->dtype);
  if (fmt == kFmtQ4K) {
    QMM_HIP(hipMemcpyAsync(t->data, src, t->bytes, hipMemcpyDeviceToDevice, s));
    return QMM_OK;
  }
  long long nblocks = t->n * (t->k / qmm_block_size(t->dtype));
  const void* a0 = src;
  void* a1 = t->data;
  int f = fmt;
  void* args[] = {&a0, &a1, &nblocks, &f};
  return launch(d, "qmm_ggml_to_dev", ceil_div(nblocks, 256), 256, 0, s, args);
}

int qmm_qtensor_from_ggml(int dtype, int64_t n, int64_t k, const void* bytes, int bytes_on_device,
                          void* stream, qmm_qtensor** out) {
  if (!out || !bytes) return fail(QMM_ERR_INVALID, "null pointer");
  *out = nullptr;
  QMM_TRY(check_shape(dtype, n, k));
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  qmm_qtensor* t;
  QMM_TRY(alloc_tensor(dtype, n, k, &t));
  const void* src = bytes;
  void* staging = nullptr;
  int rc = QMM_OK;
  if (!bytes_on_device) {
    if (fmt_of(dtype) == kFmtQ4K) {
      hipError_t e = hipMemcpyAsync(t->data, bytes, t->bytes, hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
      if (e != hipSuccess) rc = fail(QMM_ERR_HIP, "upload: %s", hipGetErrorString(e));
      if (rc != QMM_OK) {
        qmm_qtensor_free(t);
        return rc;
      }
      *out = t;
      return QMM_OK;
    }
    hipError_t e = hipMalloc(&staging, t->bytes);
    if (e != hipSuccess) {
      qmm_qtensor_free(t);
      return fail(QMM_ERR_OOM, "hipMalloc(staging %zu): %s", t->bytes, hipGetErrorString(e));
    }
    e = hipMemcpyAsync(staging, bytes, t->bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) rc = fail(QMM_ERR_HIP, "upload: %s", hipGetErrorString(e));
    src = staging;
  }
  if (rc == QMM_OK) rc = ggml_to_dev(d, t, src, s);
  if (staging) {
    hipError_t e = hipStreamSynchronize(s);
    if (rc == QMM_OK && e != hipSuccess) rc = fail(QMM_ERR_HIP, "sync: %s", hipGetErrorString(e));
    (void)hipFree(staging);
  }
  if (rc != QMM_OK) {
    qmm_qtensor_free(t);
    return rc;
  }
  *out = t;
  return QMM_OK;
}

int qmm_qtensor_quantize(int dtype, int64_t n, int64_t k, const float* w, void* stream, qmm_qtensor** out) {
  if (!out || !w) return fail(QMM_ERR_INVALID, "null pointer");
  *out = nullptr;
  QMM_TRY(check_shape(dtype, n, k));
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  qmm_qtensor* t;
  QMM_TRY(alloc_tensor(dtype, n, k, &t));
  const int fmt = fmt_of(dtype);
  long long nblocks = n * (k / qmm_block_size(dtype));
  void* ggml = t->data;
  int rc = QMM_OK;
  if (fmt != kFmtQ4K) {
    hipError_t e = hipMalloc(&ggml, t->bytes);
    if (e != hipSuccess) {
      qmm_qtensor_free(t);
      return fail(QMM_ERR_OOM, "hipMalloc(staging %zu): %s", t->bytes, hipGetErrorString(e));
    }
  }
  if (fmt == kFmtQ80) {
    // Q8_0 weights use the same from_float as Q8_0 activations: treat the
    // matrix as one row of n*k values.
    long long ld = 0;
    int kk = (int)(n * k), one = 1;
    if ((long long)kk != n * k) rc = fail(QMM_ERR_INVALID, "Q8_0 tensor too large");
    const float* x = w;
    void* args[] = {&x, &ld, &ggml, &kk, &one};
    if (rc == QMM_OK) rc = launch(d, "qmm_quantize_q8_0", ceil_div(nblocks * 8, 256), 256, 0, s, args);
  } else {
    const float* x = w;
    void* args[] = {&x, &ggml, &nblocks};
    rc = launch(d, fmt == kFmtQ4K ? "qmm_quantize_q4k_w" : "qmm_quantize_q6k_w", ceil_div(nblocks, 64), 64,
                0, s, args);
  }
  if (rc == QMM_OK && fmt != kFmtQ4K) rc = ggml_to_dev(d, t, ggml, s);
  if (fmt != kFmtQ4K) {
    hipError_t e = hipStreamSynchronize(s);
    if (rc == QMM_OK && e != hipSuccess) rc = fail(QMM_ERR_HIP, "sync: %s", hipGetErrorString(e));
    (void)hipFree(ggml);
  }
  if (rc != QMM_OK) {
    qmm_qtensor_free(t);
    return rc;
  }
  *out = t;
  return QMM_OK;
}

int qmm_qtensor_dequantize_to(const qmm_qtensor* t, void* dst, int out_dtype, void* stream) {
  if (!t || !dst) return fail(QMM_ERR_INVALID, "null pointer");
  const char* name = out_dtype == QMM_F32    ? "qmm_dequantize"
                     : out_dtype == QMM_F16  ? "qmm_dequantize_f16"
                     : out_dtype == QMM_BF16 ? "qmm_dequantize_bf16"
                                             : nullptr;
  if (!name) return fail(QMM_ERR_INVALID, "dequantize: output dtype %d (F32 = 0, F16 = 1, BF16 = 30)", out_dtype);
  Device* d;
  QMM_TRY(current_device(&d));
  const int fmt = fmt_of(t->dtype);
  long long nblocks = t->n * (t->k / qmm_block_size(t->dtype));
  const void* a0 = t->data;
  void* a1 = dst;
  int f = fmt;
  void* args[] = {&a0, &a1, &nblocks, &f};
  const long long threads = fmt == kFmtQ80 ? nblocks : nblocks * 8;
  return launch(d, name, ceil_div(threads, 256), 256, 0, (hipStream_t)stream, args);
}

int qmm_qtensor_dequantize(const qmm_qtensor* t, float* dst, void* stream) {
  return qmm_qtensor_dequantize_to(t, dst, QMM_F32, stream);
}

int qmm_qtensor_to_ggml(const qmm_qtensor* t, void* dst, int dst_on_device, void* stream) {
  if (!t || !dst) return fail(QMM_ERR_INVALID, "null pointer");
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  const int fmt = fmt_of(t->dtype);
  if (fmt == kFmtQ4K) {
    QMM_HIP(hipMemcpyAsync(dst, t->data, t->bytes, dst_on_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s));
    if (!dst_on_device) QMM_HIP(hipStreamSynchronize(s));
    return QMM_OK;
  }
  void* out = dst;
  if (!dst_on_device) {
    hipError_t e = hipMalloc(&out, t->bytes);
    if (e != hipSuccess) return fail(QMM_ERR_OOM, "hipMalloc(staging %zu): %s", t->bytes, hipGetErrorString(e));
  }
  long long nblocks = t->n * (t->k / qmm_block_size(t->dtype));
  const void* a0 = t->data;
  void* a1 = out;
  int f = fmt;
  void* args[] = {&a0, &a1, &nblocks, &f};
  int rc = launch(d, "qmm_dev_to_ggml", ceil_div(nblocks, 256), 256, 0, s, args);
  if (!dst_on_device) {
    if (rc == QMM_OK) {
      hipError_t e = hipMemcpyAsync(dst, out, t->bytes, hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
      if (e != hipSuccess) rc = fail(QMM_ERR_HIP, "download: %s", hipGetErrorString(e));
    } else {
      (void)hipStreamSynchronize(s);
    }
    (void)hipFree(out);
  }
  return rc;
}

int qmm_qtensor_info(const qmm_qtensor* t, int* dtype, int64_t* n, int64_t* k) {
  if (!t) return fail(QMM_ERR_INVALID, "null tensor");
  if (dtype) *dtype = t->dtype;
  if (n) *n = t->n;
  if (k) *k = t->k;
  return QMM_OK;
}

size_t qmm_qtensor_ggml_bytes(const qmm_qtensor* t) { return t ? t->bytes : 0; }

void qmm_qtensor_free(qmm_qtensor* t) {
  if (!t) return;
  if (t->data) {
    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != t->device) (void)hipSetDevice(t->device);
    (void)hipFree(t->data);
    if (prev != t->device) (void)hipSetDevice(prev);
  }
  delete t;
}

int qmm_quantize_rows(int vdtype, const float* x, int64_t m, int64_t k, int64_t ldx, void* xq, void* stream) {
  if (!x || !xq) return fail(QMM_ERR_INVALID, "null pointer");
  if (vdtype != QMM_Q8K && vdtype != QMM_Q8_0) return fail(QMM_ERR_INVALID, "vec-dot dtype %d is not Q8_0/Q8K", vdtype);
  const int bs = qmm_block_size(vdtype);
  if (m <= 0 || k <= 0 || k % bs) return fail(QMM_ERR_INVALID, "bad activation shape (%lld, %lld) for block size %d", (long long)m, (long long)k, bs);
  if (ldx < k) return fail(QMM_ERR_INVALID, "row stride %lld < k %lld", (long long)ldx, (long long)k);
  if (k > (1LL << 30) || m > (1LL << 30)) return fail(QMM_ERR_INVALID, "activation too large");
  Device* d;
  QMM_TRY(current_device(&d));
  long long ld = ldx;
  int kk = (int)k, mm = (int)m;
  void* args[] = {&x, &ld, &xq, &kk, &mm};
  const long long nblocks = m * (k / bs);
  if (vdtype == QMM_Q8K) return launch(d, "qmm_quantize_q8k", ceil_div(nblocks, 4), 256, 0, (hipStream_t)stream, args);
  return launch(d, "qmm_quantize_q8_0", ceil_div(nblocks * 8, 256), 256, 0, (hipStream_t)stream, args);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Plane layout of m activation rows for the GEMM: int8 q8 [m][k], f32 scales
// [m][k/block], int16 32-element sums [m][k/256][8] (k-quants).
struct Planes {
  size_t q8, d, s, total;
};
static Planes mmq_planes(int dtype, int64_t m, int64_t k) {
  Planes p;
  const int64_t nbd = dtype == QMM_Q8_0 ? k / 32 : k / 256;
  p.q8 = 0;
  p.d = align256((size_t)(m * k));
  p.s = p.d + align256((size_t)(m * nbd) * 4);
  p.total = p.s + (dtype == QMM_Q8_0 ? 0 : align256((size_t)(m * (k / 256)) * 16));
  return p;
}

// The GEMM handles m > 8 rows when k is a whole number of 256-wide steps.
static bool use_gemm(const qmm_qtensor* w, int64_t m) { return m > 8 && w->k % 256 == 0; }

static size_t gemm_split_bytes(const qmm_qtensor* w, int64_t m);

size_t qmm_matmul_workspace_size(const qmm_qtensor* w, int64_t m) {
  if (!w || m <= 0) return 0;
  const int vt = qmm_vec_dot_type(w->dtype);
  const size_t ggml = (size_t)m * (size_t)(w->k / qmm_block_size(vt)) * qmm_type_size(vt);
  if (!use_gemm(w, m)) return ggml;
  // activation planes, then the split-K partials
  return mmq_planes(w->dtype, m, w->k).total + gemm_split_bytes(w, m);
}

// Job table of one GEMV launch (passed to the kernel as scalar arguments).
constexpr int kMaxJobs = 8;  // the kernels' qmm::kMaxJobs

struct GemvJobs {
  const void* wq[kMaxJobs];
  float* y[kMaxJobs];
  int rows[kMaxJobs];
  int ldy[kMaxJobs];
  int row0[kMaxJobs];
  int trows[kMaxJobs];
  int njobs;
  int total;
};

struct GemvTarget {
  const qmm_qtensor* w;
  float* y;
  int64_t ldy;
};

// GEMV launch for m <= 8 activation rows over up to kMaxJobs weights (same dtype
// and k) sharing one activation. `act` is m rows of quantized blocks, or f32
// rows with stride ldx when `fused` (then the kernel quantizes in its prologue).
static int gemv(Device* d, const GemvTarget* tg, int count, const void* act, bool fused, int64_t ldx, int m,
                int* dump, hipStream_t s, const float* norm_w = nullptr, float eps = 0.0f, int accumulate = 0,
                bool silu = false) {
  if (count > 4 && m != 1) {  // eight-job kernels exist for m == 1 only: two launches
    QMM_TRY(gemv(d, tg, 4, act, fused, ldx, m, dump, s, norm_w, eps, accumulate));
    return gemv(d, tg + 4, count - 4, act, fused, ldx, m, dump, s, norm_w, eps, accumulate);
  }
  // Q4_K and Q6_K jobs together (both take Q8_K activations): one launch of
  // the mixed one-row kernels, Q4_K jobs first (global rows >= mix_row are
  // Q6_K); other shapes take one launch per format.
  int n4 = 0, n6 = 0;
  for (int j = 0; j < count; ++j) {
    const int f = fmt_of(tg[j].w->dtype);
    n4 += f == kFmtQ4K;
    n6 += f == kFmtQ6K;
  }
  const bool mixed = n4 > 0 && n6 > 0;
  if (mixed && n4 + n6 != count) return fail(QMM_ERR_INVALID, "only Q4_K and Q6_K weights share a launch");
  GemvTarget sorted[kMaxJobs];
  int mix_row = 0;
  if (mixed) {
    int a = 0, b = n4;
    for (int j = 0; j < count; ++j) {
      if (fmt_of(tg[j].w->dtype) == kFmtQ4K) {
        sorted[a++] = tg[j];
        mix_row += (int)tg[j].w->n;
      } else {
        sorted[b++] = tg[j];
      }
    }
    if (m != 1 || dump || silu) {
      QMM_TRY(gemv(d, sorted, n4, act, fused, ldx, m, dump, s, norm_w, eps, accumulate, silu));
      return gemv(d, sorted + n4, n6, act, fused, ldx, m, dump, s, norm_w, eps, accumulate, silu);
    }
    tg = sorted;
  }
  const qmm_qtensor* w = tg[0].w;
  const int fmt = fmt_of(w->dtype);
  const int nb = (int)(w->k / qmm_block_size(w->dtype));
  const int lpb = fmt == kFmtQ80 ? 1 : 4;  // lanes per weight block
  const int bpi = 64 / lpb;                // blocks per wave iteration
  const int niter = (nb + bpi - 1) / bpi;
  const int xbb = fmt == kFmtQ80 ? 36 : 292;  // LDS bytes per staged activation block
  const unsigned lds = (unsigned)(m * nb * xbb * (mixed ? 2 : 1));  // mixed: Q4_K and Q6_K layouts
  if ((int)lds > d->max_lds)
    return fail(QMM_ERR_UNSUPPORTED, "activation of %d rows x %lld needs %u B of LDS (> %d)", m, (long long)w->k, lds,
                d->max_lds);
  // 2..8 staged activation rows of one k-quant weight: the token-interleaved
  // kernel the expert GEMV uses (one transposed reduction for all rows, no
  // per-row branches), the same bits as the general multi-row GEMV. From
  // sweeps (graph replays): m = 8 gate 14336x4096 17.4 vs 27.9 us, down
  // 4096x14336 21.4 vs 36.0 us, q 4096x4096 6.9 vs 11.6 us; m = 3 11.6 vs
  // 12.6, 15.0 vs 20.5, 5.1 vs 5.9 us. On 1024-row weights its smaller grid
  // loses below seven rows (k 1024x4096 at m = 2: 3.94 vs 3.55 us), so
  // weights under 2048 rows take it from m = 7. QMM_GEMV_ROWS=<m> takes it
  // from m rows at every size (0: never).
  int rows_from = w->n >= 2048 ? 2 : 7;
  if (const char* e = env(kEnvGemvRows)) rows_from = atoi(e);
  const unsigned long long rbody = fmt == kFmtQ4K ? 144 : 208;  // device block bodies (Q6_K's f16 d kept apart)
  // 6..8 staged rows of a Q4_K weight of >= 8192 rows: the multi-token GEMV
  // on the int8 matrix cores (qmm_gemv_rowsm_q4k: 16 rows x 16 tokens per
  // MFMA, the activation read once per workgroup instead of once per token
  // and weight slice). From the sweep at 14336 x 4096 (kernel time): m = 8
  // 13.9 vs 18.9 us for the token-interleaved kernel, m = 4 about even; its
  // fixed cost per weight slice loses below six rows. QMM_GEMVM=0 never, 1
  // wherever it applies (2..8 rows of Q4_K).
  int gvm = -1;
  if (const char* e = env(kEnvGemvm)) gvm = atoi(e);
  if (count == 1 && !fused && !silu && dump == nullptr && fmt == kFmtQ4K && m >= 2 && m <= 8 && nb <= 64 &&
      (unsigned long long)w->n * nb * rbody < (1ull << 32) &&
      (gvm > 0 || (gvm < 0 && m >= 6 && w->n >= 8192))) {
    const void* wq = w->data;
    float* yy = tg[0].y;
    int ldy = (int)tg[0].ldy, mm = m, K = (int)w->k, N = (int)w->n, acc = accumulate;
    void* args[] = {&wq, &yy, &ldy, &act, &mm, &K, &N, &acc};
    const long long groups = (N + 15) / 16;  // 16 weight rows per wave, four waves per workgroup
    return launch(d, "qmm_gemv_rowsm_q4k_w4_p4", ceil_div(groups, 4), 256, (unsigned)(m * (K + 16) + 320 * nb), s,
                  args);
  }
  if (count == 1 && !fused && !silu && dump == nullptr && rows_from > 0 && m >= rows_from && m <= 8 &&
      fmt != kFmtQ80 && nb <= 64 && (unsigned long long)w->n * nb * rbody < (1ull << 32)) {
    char rname[32];
    snprintf(rname, sizeof(rname), "qmm_gemv_rows_%s", fmt_name(fmt));
    const void* wq = w->data;
    float* yy = tg[0].y;
    int ldy = (int)tg[0].ldy, mm = m, K = (int)w->k, N = (int)w->n, acc = accumulate;
    void* args[] = {&wq, &yy, &ldy, &act, &mm, &K, &N, &acc};
    const long long grid = std::min<long long>((long long)d->num_cu * 2, (N + 15) / 16);
    return launch(d, rname, (unsigned)grid, 1024, (unsigned)(m * nb * 292), s, args);
  }
  GemvJobs jobs = {};
  long long total = 0;
  for (int j = 0; j < count; ++j) {
    jobs.wq[j] = tg[j].w->data;
    jobs.y[j] = tg[j].y;
    jobs.rows[j] = (int)tg[j].w->n;
    jobs.ldy[j] = (int)tg[j].ldy;
    jobs.row0[j] = 0;
    jobs.trows[j] = (int)tg[j].w->n;
    total += tg[j].w->n;
  }
  if (total > (1LL << 31) - 1) return fail(QMM_ERR_INVALID, "too many output rows in one launch");
  jobs.njobs = count;
  jobs.total = (int)total;
  // Launch shape (from sweeps on MI355X at the Llama-3-8B decode shapes).
  // Each wave keeps one or two weight slices per lane in flight and prefetches
  // its next row while finishing the current one; 16 waves are resident per
  // CU. Fused (in-kernel quantization) and long-K staged launches use one
  // 16-wave workgroup per CU: the workgroup shares its activation over more
  // rows, and a grid that leaves some CUs with one workgroup more than others
  // finishes with those CUs (up to 35% slower at the gate/up and head shapes).
  // Staged launches with a short activation (<= 8 KB in LDS) use 4-wave
  // workgroups, so that even 1024-row weights spread over every CU. m > 1
  // staged launches use 8 waves (the 16-wave variants would exceed 128 VGPRs).
  int wv = 16, r = 1, u = 1;
  if (!fused) {
    if (m > 1) {
      wv = 8;
      if (niter >= 2) u = 2;
    } else if (nb * xbb <= 8192) {
      wv = 4;
    }
  }
  int waves_per_cu = !fused && m > 1 ? 20 : 16;  // m > 1: the earlier sweep's optimum
  const Tuning& tu = tuning();
  if (tu.w > 0 && tu.r > 0 && tu.u > 0) { wv = tu.w; r = tu.r; u = tu.u; }
  if (tu.waves_per_cu > 0) waves_per_cu = tu.waves_per_cu;
  // more than four weights: the eight-job kernels (M = 1; r = u = 1 shapes)
  const int jcap = count > 4 ? kMaxJobs : 4;
  if (jcap > 4) {  // instantiated: staged w4/w8/w16, fused w8/w16; r 1..2, u 1
    u = 1;
    if (r > 2) r = 2;
    if (fused && wv < 8) wv = 8;
  }
  // One activation row without a block-dot dump: the lean one-row kernels
  // (gemv1: activation slice kept in registers, one row per wave at a time).
  const bool one = m == 1 && dump == nullptr && r == 1 && u == 1 && (wv == 4 || wv == 8 || wv == 16) &&
                   tu.gemv1 != 0;
  // k-quant weights with an activation of at most 64 blocks (K <= 16384):
  // the prefetch-ring kernels (gemv1p), one 16-wave workgroup per CU; their
  // prologue stages one activation item per thread. From sweeps at the decode
  // shapes they beat gemv1 for Q6_K rows of several slices (down 4096x14336:
  // 13.2 vs 13.9 us staged, 15.4 vs 16.1 fused, two slices in flight) and for
  // staged Q4_K launches of one row per wave (q 4096x4096: 4.8 vs 5.1 us);
  // gemv1 keeps the rest. QMM_GEMV1P=<P> forces them (0: never).
  const long long rows_cu = (long long)d->num_cu * 16;
  bool ring = m == 1 && dump == nullptr && fmt != kFmtQ80 && nb <= 64 && tu.gemv1p != 0 && !silu &&
              !(tu.w > 0 && tu.r > 0 && tu.u > 0);
  if (ring && tu.gemv1p < 0)
    ring = !mixed && ((fmt == kFmtQ6K && niter >= 2) ||
                      (fmt == kFmtQ4K && !fused && total > rows_cu / 4 && total <= rows_cu));
  char name[80];
  if (ring) {
    wv = 16;
    waves_per_cu = 16;
    // prefetch depth (instantiated: Q4_K 1, 2, 4; Q6_K and mixed 1, 2, 3)
    int pd = fmt == kFmtQ4K ? 1 : 2;
    if (tu.gemv1p > 0) {
      pd = std::min(tu.gemv1p, fmt == kFmtQ4K && !mixed ? 4 : 3);
      if (fmt == kFmtQ4K && !mixed && pd == 3) pd = 2;
    }
    snprintf(name, sizeof(name), "qmm_gemv1p%s_%s_w16_p%d%s", fused ? "f" : "", mixed ? "q4k6k" : fmt_name(fmt), pd,
             jcap > 4 ? "_j8" : "");
  } else if (silu) {
    // silu(g) * u in the prologue: one-row kernels with a four-job table, 8 or 16 waves
    if (!fused || m != 1 || dump || count > 4) return fail(QMM_ERR_INVALID, "silu prologue needs one fused row");
    wv = wv >= 16 ? 16 : 8;
    r = u = 1;
    snprintf(name, sizeof(name), "qmm_gemv1s_%s_w%d", fmt_name(fmt), wv);
  } else if (one)
    snprintf(name, sizeof(name), "qmm_gemv1%s_%s_w%d%s", fused ? "f" : "", mixed ? "q4k6k" : fmt_name(fmt), wv,
             jcap > 4 ? "_j8" : "");
  else if (mixed) {  // tuned to a shape without mixed kernels: one launch per format
    QMM_TRY(gemv(d, tg, n4, act, fused, ldx, m, dump, s, norm_w, eps, accumulate, silu));
    return gemv(d, tg + n4, n6, act, fused, ldx, m, dump, s, norm_w, eps, accumulate, silu);
  } else
    snprintf(name, sizeof(name), "qmm_gemv%s_%s_m%d_w%d_r%d_u%d%s", fused ? "f" : "", fmt_name(fmt), m, wv, r, u,
             jcap > 4 ? "_j8" : "");
  long long wgs = (total + wv * r - 1) / (wv * r);
  const long long cap = ((long long)d->num_cu * waves_per_cu + wv - 1) / wv;
  if (wgs > cap) wgs = cap;
  const void* a = act;
  long long lx = ldx;
  int K = (int)w->k;
  int* dp = dump;
  void* args[6 * kMaxJobs + 10];
  int na = 0;
  for (int j = 0; j < jcap; ++j) {
    args[na++] = &jobs.wq[j];
    args[na++] = &jobs.y[j];
    args[na++] = &jobs.rows[j];
    args[na++] = &jobs.ldy[j];
    args[na++] = &jobs.row0[j];
    args[na++] = &jobs.trows[j];
  }
  args[na++] = &jobs.njobs;
  args[na++] = &jobs.total;
  args[na++] = &a;
  args[na++] = &lx;
  args[na++] = &K;
  args[na++] = &dp;
  args[na++] = &norm_w;
  args[na++] = &eps;
  args[na++] = &accumulate;
  if (mixed) args[na++] = &mix_row;
  return launch(d, name, (unsigned)wgs, 64 * wv, lds, s, args);
}

// Kernel, tile and split-K plan of one prefill GEMM.
struct GemmPlan {
  char name[40];
  unsigned gx, gy, threads, lds;
  int splits, kc;  // K steps per split
  int sk_tiles;    // > 0: the stream-K schedule (qmm_mmqs_q4k_sk) over a grid of gx workgroups
  int tiles, mtiles;
};

// Split-K: a grid of fewer than half as many tiles as CUs (e.g. m = 127
// against N = 4096: 32-64 tiles) leaves most CUs idle for the whole K loop;
// splitting the K steps over blockIdx.z fills them, and a small kernel sums
// the splits' f32 partials in split order. The count minimises (rounds of
// the grid over the resident workgroup slots) x (K steps per split), with at
// least two K steps per split (one-step splits spend more on writing and
// re-reading their partials than they gain) and the smaller count on a tie.
// Slots are CUs times the workgroups whose LDS fits in one CU. Per call at
// m = 127 (quantization, GEMM and sum), against one split per CU / tiles:
// gate 14336x4096 Q4_K 45.7 -> 36.6 us (2 splits, not 3: 336 one-per-CU
// workgroups ran a second, mostly empty round), Q6_K down 4096x14336
// 69.3 -> 57.3 us (8, not 4: its 60 KB tile fits twice per CU), k 1024x4096
// 19.0 -> 17.5 us (8, not 16). QMM_SPLITK=0 disables it, QMM_SPLITK=<S>
// forces S splits.
static constexpr unsigned kMmqStaticLds = 61440;  // the first-generation tile's static LDS (MmqLds)
// one LDS stage of the split-digit Q6_K tile (mmqs6): activation rows, int8
// codes, digit bytes, column d, row scales (128 x 256, 128 x 256, 128 x 48,
// 128 x 4, 128 x 4 bytes)
static constexpr unsigned kS6StageBytes = 128 * 256 + 128 * 256 + 128 * 48 + 128 * 4 + 128 * 4;
// one LDS stage of the split-scale Q4_K tile (mmqs): activation rows, weight
// quants, block headers, row scales, A' and B' rows, split-scale multipliers
// (the kernels' SLayout<false>::kStage; DUMP adds 128 x 16 bytes of sums)
static constexpr unsigned kSStageBytes = 128 * 256 + 128 * 128 + 128 * 16 + 128 * 4 + 128 * 48 + 128 * 48 + 128 * 80;
// One LDS stage of the Q8_0 tile (mmqs8): activation rows, weight codes, f32
// weight and activation block scales (the kernels' kS8Stage).
static constexpr unsigned kS8StageBytes = 128 * 256 + 128 * 256 + 128 * 32 + 8 * 128 * 4;
static constexpr int kMmqBMRows = 64;             // and its M tile
static void plan_splits(const Device* d, GemmPlan& p, int nbk) {
  const long long tiles = (long long)p.gx * p.gy;
  int sp = 1;
  if (const char* e = env(kEnvSplitK)) {
    sp = atoi(e);
  } else if (tiles * 2 <= d->num_cu) {
    const unsigned lds = p.lds ? p.lds : kMmqStaticLds;
    const long long slots = (long long)d->num_cu * std::max(1u, (unsigned)d->max_lds / lds);
    long long best = -1;
    for (int c = 1; c <= std::min(16, nbk); ++c) {
      const int kc = (nbk + c - 1) / c;
      if (c > 1 && kc < 2) break;
      const long long cost = (tiles * c + slots - 1) / slots * kc;
      if (best < 0 || cost < best) {
        best = cost;
        sp = c;
      }
    }
  }
  sp = std::max(1, std::min(std::min(sp, 16), nbk));
  p.kc = (nbk + sp - 1) / sp;
  p.splits = (nbk + p.kc - 1) / p.kc;
}

// Stream-K (mmqs, one 512-thread workgroup per CU; opt-in, QMM_STREAMK=1):
// a grid of T tiles that is not a whole number of rounds over the CUs
// (config 4's gate 14336x4096 at M = 512: 448 tiles, 1.75 rounds, a quarter
// of the CUs idle in the second) runs as floor rounds of data-parallel tiles
// plus the rest as stream-K tiles whose (tile, K step) iterations are cut
// into equal ranges, one per CU (qmm_mmqs_q4k_sk). The stream-K part is the
// remainder r = T % G, or r + G when r tiles would give a CU fewer than
// max(2, nbk / 2) K steps; a grid of fewer than G tiles is all stream-K
// (in place of split-K). Below two K steps per CU the plain plan stays.
// Measured at M = 512 it is no faster than the plain grid: the schedule
// without its partial fixup takes 97.5 us at the gate shape against 105.9 us
// for the plain 1.75 rounds, and the fixup's dependent store / counter /
// load round trips at the end of the split tiles give the difference back
// (106.0 us; the down shape 106.9 us against 106.4 us with split-K), so it is
// not the default. A forced QMM_SPLITK also turns it off.
static void plan_streamk(const Device* d, GemmPlan& p, int nbk) {
  p.sk_tiles = 0;
  p.tiles = (int)(p.gx * p.gy);
  p.mtiles = (int)p.gy;
  const char* e = env(kEnvStreamK);
  if (e == nullptr || atoi(e) == 0 || env(kEnvSplitK) != nullptr) return;
  const int G = d->num_cu, T = p.tiles;
  if (G < 8 || G % 8 != 0 || T % G == 0) return;
  int sk = T < G ? T : T % G;
  if (T > G && (long long)sk * nbk < (long long)G * std::max(2, nbk / 2)) sk += G;
  if ((long long)sk * nbk < 2LL * G) return;
  p.sk_tiles = sk;
  p.gx = (unsigned)G;
  p.gy = 1;
  p.splits = 1;
  p.kc = nbk;
}

// Scratch of the stream-K schedule: the partial slots (two 128 x 128 f32
// tiles per workgroup), then the stream-K tiles' counters.
static size_t streamk_bytes(const GemmPlan& p) {
  return p.sk_tiles > 0 ? align256((size_t)2 * p.gx * 128 * 128 * 4) + align256((size_t)p.sk_tiles * 4) : 0;
}

static GemmPlan gemm_plan(const Device* d, const qmm_qtensor* w, int64_t m, bool dump) {
  GemmPlan p;
  p.sk_tiles = 0;
  const int fmt = fmt_of(w->dtype);
  const int M = (int)m, N = (int)w->n;
  // Q4_K: the second-generation kernel, 128x128 tiles (one workgroup of 512
  // threads per CU, double-buffered LDS of 2 x 58 KB). QMM_MMQ2="BM,BN" picks
  // 64-row tiles instead.
  int bm = 128, bn = 128;
  if (const char* e = env(kEnvMmq2)) {
    int a = 0, b = 0;
    if (sscanf(e, "%d,%d", &a, &b) == 2 && (a == 64 || a == 128) && (b == 64 || b == 128) && !(a == 128 && b == 64)) {
      bm = a;
      bn = b;
    }
  }
  const unsigned lds2 = (unsigned)(2 * (bm * 272 + bn * 144 + bm * 4 + bm * 16));
  // Q4_K: mmq2 (128x128 tiles, 8 waves, VALU sub-block scaling) when its grid
  // covers at least half the CUs (split-K fills the rest: 4096x14336 at
  // M = 512, 128 tiles x 2 splits: 120 us); below that (the prefill's
  // M = 127) the split-scale mmq4 with 128x64 tiles (4 waves, one per SIMD),
  // twice the workgroups (14336x4096 at M = 127: 41 vs 52 us).
  // QMM_MMQ=2 / QMM_MMQ=4 force one; QMM_MMQ4_BN=128 picks 128x128 mmq4 tiles.
  const char* gen = env(kEnvMmq);
  const long long tiles2 = (long long)((N + bn - 1) / bn) * ((M + bm - 1) / bm);
  const bool use4 = gen ? atoi(gen) == 4 : tiles2 * 2 < d->num_cu;
  // Q4_K default: mmqs (split-scale d term on int8 MFMA, mins term on bf16
  // MFMA, 128 x 128 tiles of eight waves, two per SIMD, LDS 2 x 72.5 KB);
  // QMM_MMQ=2 / 4 select the older generations
  const unsigned ldss = 2u * (kSStageBytes + (dump ? 128 * 16 : 0));
  if (fmt == kFmtQ4K && gen == nullptr && (int)ldss <= d->max_lds) {
    snprintf(p.name, sizeof(p.name), "qmm_mmqs_q4k%s", dump ? "_dump" : "");
    p.gx = (unsigned)((N + 127) / 128);
    p.gy = (unsigned)((M + 127) / 128);
    p.threads = 512;
    p.lds = ldss;
  } else if (fmt == kFmtQ4K && use4) {
    int b4 = 64;
    if (const char* e = env(kEnvMmq4Bn)) b4 = atoi(e) == 128 ? 128 : 64;
    snprintf(p.name, sizeof(p.name), "qmm_mmq4_q4k_n%d%s", b4, dump ? "_dump" : "");
    p.gx = (unsigned)((N + b4 - 1) / b4);
    p.gy = (unsigned)((M + 127) / 128);
    p.threads = 256;
    p.lds = (unsigned)(2 * (128 * 272 + b4 * 144 + 128 * 4 + 128 * 16));
  } else if (fmt == kFmtQ6K && env(kEnvMmq6) == nullptr && (int)(2 * kS6StageBytes) <= d->max_lds) {
    // Q6_K default: mmqs6 (the sub-block scales as three signed digits in the int8 MFMA operands, 128 x 128
    // tiles of eight waves, LDS 2 x 71 KB); QMM_MMQ6=1 selects the first-generation tile
    snprintf(p.name, sizeof(p.name), "qmm_mmqs6_q6k%s", dump ? "_dump" : "");
    p.gx = (unsigned)((N + 127) / 128);
    p.gy = (unsigned)((M + 127) / 128);
    p.threads = 512;
    p.lds = 2 * kS6StageBytes;
  } else if (fmt == kFmtQ80 && env(kEnvMmq8) == nullptr && (int)(2 * kS8StageBytes) <= d->max_lds) {
    // Q8_0 default: mmqs8 (both operands straight into LDS, 128 x 128 tiles of eight waves, LDS 2 x 72 KB);
    // QMM_MMQ8=1 selects the first-generation tile
    snprintf(p.name, sizeof(p.name), "qmm_mmqs8_q8_0%s", dump ? "_dump" : "");
    p.gx = (unsigned)((N + 127) / 128);
    p.gy = (unsigned)((M + 127) / 128);
    p.threads = 512;
    p.lds = 2 * kS8StageBytes;
  } else if (fmt == kFmtQ4K && (int)lds2 <= d->max_lds && env(kEnvMmq1) == nullptr) {
    snprintf(p.name, sizeof(p.name), "qmm_mmq2_q4k_m%d_n%d%s", bm, bn, dump ? "_dump" : "");
    p.gx = (unsigned)((N + bn - 1) / bn);
    p.gy = (unsigned)((M + bm - 1) / bm);
    p.threads = (unsigned)(bm * bn / 32);
    p.lds = lds2;
  } else {
    snprintf(p.name, sizeof(p.name), "qmm_mmq_%s%s", fmt_name(fmt), dump ? "_dump" : "");
    p.gx = (unsigned)((N + 127) / 128);
    p.gy = (unsigned)((M + 63) / 64);
    p.threads = 256;
    p.lds = 0;
  }
  p.tiles = (int)(p.gx * p.gy);
  p.mtiles = (int)p.gy;
  if (fmt == kFmtQ4K && gen == nullptr && !dump && p.threads == 512) plan_streamk(d, p, (int)(w->k / 256));
  if (p.sk_tiles == 0) plan_splits(d, p, (int)(w->k / 256));
  return p;
}

// Scratch bytes gemm() of w at m rows uses: f32 split partials, or the
// stream-K schedule's partial slots and counters (0 for neither).
static size_t gemm_split_bytes(const qmm_qtensor* w, int64_t m) {
  Device* d;
  if (current_device(&d) != QMM_OK) return 0;
  const GemmPlan p = gemm_plan(d, w, m, false);
  if (p.sk_tiles > 0) return streamk_bytes(p);
  return p.splits > 1 ? align256((size_t)p.splits * (size_t)m * (size_t)w->n * 4) : 0;
}

// The stream-K scratch of w's plan at m rows (0 when it is not stream-K):
// the callers that keep split partials of their own size it separately.
static size_t gemm_sk_bytes(const Device* d, const qmm_qtensor* w, int64_t m) {
  return streamk_bytes(gemm_plan(d, w, m, false));
}

// The GEMM kernel of plan p over activation planes at `ws` (see mmq_planes):
// unsplit, into y (row stride ldy, accumulate as asked); split, the f32
// partials [p.splits][m][n] into `part` and nothing summed.
static int gemm_launch(Device* d, const qmm_qtensor* w, const uint8_t* ws, int64_t m, const GemmPlan& p, float* y,
                       int64_t ldy, int* dump, hipStream_t s, int accumulate, float* part, void* sk_scratch) {
  const Planes pl = mmq_planes(w->dtype, m, w->k);
  if ((uintptr_t)ws % 16) return fail(QMM_ERR_INVALID, "GEMM workspaces must be 16-byte aligned");
  const bool split = p.splits > 1;
  const void* wq = w->data;
  const void* q8 = ws + pl.q8;
  const void* dd = ws + pl.d;
  const void* ss = ws + pl.s;
  if (p.sk_tiles > 0) {
    // stream-K: the counters cleared by a kernel (never a memset: callers capture this into graphs), then the
    // GEMM into y
    if (sk_scratch == nullptr) return fail(QMM_ERR_INVALID, "stream-K GEMM without scratch");
    float* slots = (float*)sk_scratch;
    unsigned* counters = (unsigned*)((uint8_t*)sk_scratch + align256((size_t)2 * p.gx * 128 * 128 * 4));
    int nc = p.sk_tiles;
    void* za[] = {&counters, &nc};
    QMM_TRY(launch(d, "qmm_zero_u32", (unsigned)std::min(64, (nc + 255) / 256), 256, 0, s, za));
    int M = (int)m, N = (int)w->n, K = (int)w->k, ld = (int)ldy, acc = accumulate;
    int gy = p.mtiles, T = p.tiles, sk = p.sk_tiles;
    void* args[] = {&wq, &q8, &dd, &ss, &y, &M, &N, &K, &ld, &acc, &gy, &T, &sk, &slots, &counters};
    return launch(d, "qmm_mmqs_q4k_sk", p.gx, p.threads, p.lds, s, args);
  }
  float* yy = split ? part : y;
  int M = (int)m, N = (int)w->n, K = (int)w->k, ld = split ? N : (int)ldy;
  int* dp = dump;
  int acc = split ? 0 : accumulate;
  // XCD-aware tile order (QMM_MMQ_XCD=0: plain blockIdx order); split
  // launches keep the plain order
  int remap = split ? 0 : 1;
  if (const char* e = env(kEnvMmqXcd)) remap = remap && atoi(e) != 0;
  int kc = p.kc;
  long long ysplit = split ? (long long)M * N : 0;
  void* args[] = {&wq, &q8, &dd, &ss, &yy, &M, &N, &K, &ld, &dp, &acc, &remap, &kc, &ysplit};
  hipFunction_t f;
  QMM_TRY(kernel(d, p.name, &f));
  QMM_HIP(hipModuleLaunchKernel(f, p.gx, p.gy, (unsigned)p.splits, p.threads, 1, 1, p.lds, s, args, nullptr));
  return QMM_OK;
}

// The plan of w at m rows, run unsplit when its partials would not fit in
// part_bytes.
static GemmPlan gemm_plan_fit(Device* d, const qmm_qtensor* w, int64_t m, bool dump, const float* part,
                              size_t part_bytes) {
  GemmPlan p = gemm_plan(d, w, m, dump);
  if (p.sk_tiles > 0 && (part == nullptr || streamk_bytes(p) > part_bytes)) {
    // no room for the stream-K scratch: the tile grid, split over K when that fits
    p.sk_tiles = 0;
    p.gx = (unsigned)((w->n + 127) / 128);
    p.gy = (unsigned)((m + 127) / 128);
    plan_splits(d, p, (int)(w->k / 256));
  }
  const size_t need = (size_t)p.splits * (size_t)m * (size_t)w->n * 4;
  if (p.splits > 1 && (part == nullptr || need > part_bytes)) {
    p.splits = 1;
    p.kc = (int)(w->k / 256);
  }
  return p;
}

// Prefill GEMM over activation planes at `ws` (see mmq_planes); `part` holds
// part_bytes of scratch for split partials (a split plan that does not fit
// runs as one split), which qmm_splitk_sum then adds into y.
static int gemm(Device* d, const qmm_qtensor* w, const uint8_t* ws, int64_t m, float* y, int64_t ldy, int* dump,
                hipStream_t s, int accumulate, float* part, size_t part_bytes) {
  const GemmPlan p = gemm_plan_fit(d, w, m, dump != nullptr, part, part_bytes);
  QMM_TRY(gemm_launch(d, w, ws, m, p, y, ldy, dump, s, accumulate, part, part));
  if (p.splits > 1) {
    int M = (int)m, N = (int)w->n;
    const float* pp = part;
    int sp = p.splits, lo = (int)ldy;
    void* a2[] = {&pp, &sp, &M, &N, &y, &lo, &accumulate};
    QMM_TRY(launch(d, "qmm_splitk_sum", ceil_div((int64_t)M * N, 256), 256, 0, s, a2));
  }
  return QMM_OK;
}

// f32 activations -> planes (quantized as VecDotType::from_float).
static int quantize_planes(Device* d, int wdtype, const float* x, int64_t m, int64_t k, int64_t ldx, uint8_t* ws,
                           hipStream_t s) {
  const Planes pl = mmq_planes(wdtype, m, k);
  long long ld = ldx;
  int kk = (int)k, mm = (int)m;
  void* q8 = ws + pl.q8;
  void* dd = ws + pl.d;
  void* ss = ws + pl.s;
  if (wdtype == QMM_Q8_0) {
    void* args[] = {&x, &ld, &q8, &dd, &kk, &mm};
    return launch(d, "qmm_quantize_q8_0_mmq", ceil_div(m * (k / 32) * 8, 256), 256, 0, s, args);
  }
  void* args[] = {&x, &ld, &q8, &dd, &ss, &kk, &mm};
  return launch(d, "qmm_quantize_q8k_mmq", ceil_div(m * (k / 256), 4), 256, 0, s, args);
}

// GGML vec-dot blocks -> planes.
static int blocks_to_planes(Device* d, int wdtype, const void* xq, int64_t m, int64_t k, uint8_t* ws,
                            hipStream_t s) {
  const Planes pl = mmq_planes(wdtype, m, k);
  void* q8 = ws + pl.q8;
  void* dd = ws + pl.d;
  void* ss = ws + pl.s;
  int kk = (int)k, mm = (int)m, is_q8k = wdtype == QMM_Q8_0 ? 0 : 1;
  void* args[] = {&xq, &q8, &dd, &ss, &kk, &mm, &is_q8k};
  const unsigned grid = is_q8k ? ceil_div(m * (k / 256), 4) : ceil_div(m * (k / 32), 256);
  return launch(d, "qmm_q8_blocks_to_planes", grid, 256, 0, s, args);
}

static int check_matmul(const qmm_qtensor* w, int64_t m, const float* y, int64_t ldy) {
  if (!w || !y) return fail(QMM_ERR_INVALID, "null pointer");
  if (m <= 0) return fail(QMM_ERR_INVALID, "m = %lld must be positive", (long long)m);
  if (ldy < w->n) return fail(QMM_ERR_INVALID, "output row stride %lld < n %lld", (long long)ldy, (long long)w->n);
  if (ldy > (1LL << 31) - 1) return fail(QMM_ERR_INVALID, "output row stride too large");
  int dev = 0;
  QMM_HIP(hipGetDevice(&dev));
  if (dev != w->device) return fail(QMM_ERR_INVALID, "tensor lives on device %d, current device is %d", w->device, dev);
  return QMM_OK;
}

size_t qmm_matmul_q_workspace_size(const qmm_qtensor* w, int64_t m) {
  if (!w || m <= 0 || !use_gemm(w, m)) return 0;
  return mmq_planes(w->dtype, m, w->k).total + gemm_split_bytes(w, m);
}

// m > 8 rows of GGML vec-dot blocks -> GEMM planes in the caller's
// workspace, then the GEMM (dump != nullptr: the block-dot variant).
static int gemm_from_blocks(Device* d, const qmm_qtensor* w, const void* xq, int64_t m, float* y, int64_t ldy,
                            int* dump, void* ws, size_t ws_bytes, hipStream_t s) {
  if (!use_gemm(w, m)) return fail(QMM_ERR_UNSUPPORTED, "the GEMM path (m > 8) needs k %% 256 == 0");
  const size_t pb = mmq_planes(w->dtype, m, w->k).total;
  if (!ws || ws_bytes < pb)
    return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed (qmm_matmul_q_workspace_size)", ws ? ws_bytes : 0,
                qmm_matmul_q_workspace_size(w, m));
  uint8_t* b = (uint8_t*)ws;
  QMM_TRY(blocks_to_planes(d, w->dtype, xq, m, w->k, b, s));
  // split-K partials in the rest (a plan that does not fit runs unsplit)
  return gemm(d, w, b, m, y, ldy, dump, s, 0, (float*)(b + pb), ws_bytes - pb);
}

int qmm_matmul_q(const qmm_qtensor* w, const void* xq, int64_t m, float* y, int64_t ldy, void* ws, size_t ws_bytes,
                 void* stream) {
  QMM_TRY(check_matmul(w, m, y, ldy));
  if (!xq) return fail(QMM_ERR_INVALID, "null activation");
  Device* d;
  QMM_TRY(current_device(&d));
  const int vt = qmm_vec_dot_type(w->dtype);
  if (use_gemm(w, m)) return gemm_from_blocks(d, w, xq, m, y, ldy, nullptr, ws, ws_bytes, (hipStream_t)stream);
  const size_t xrow = (size_t)(w->k / qmm_block_size(vt)) * qmm_type_size(vt);
  // Rows are processed in groups of up to 8 by the GEMV.
  for (int64_t m0 = 0; m0 < m; m0 += 8) {
    const int mm = (int)(m - m0 < 8 ? m - m0 : 8);
    GemvTarget t = {w, y + m0 * ldy, ldy};
    QMM_TRY(gemv(d, &t, 1, (const uint8_t*)xq + m0 * xrow, false, 0, mm, nullptr, (hipStream_t)stream));
  }
  return QMM_OK;
}

// Weights that can share one activation in a call: the same k, and the same
// dtype or both Q4_K / Q6_K (whose activations are both Q8_K).
static bool same_act(const qmm_qtensor* a, const qmm_qtensor* b) {
  if (a->k != b->k) return false;
  if (a->dtype == b->dtype) return true;
  const bool ka = a->dtype == QMM_Q4K || a->dtype == QMM_Q6K, kb = b->dtype == QMM_Q4K || b->dtype == QMM_Q6K;
  return ka && kb;
}

int qmm_matmul_multi_q(const qmm_qtensor* const* w, int count, const void* xq, int64_t m, float* const* y,
                       const int64_t* ldy, void* ws, size_t ws_bytes, void* stream) {
  if (!w || !y || !ldy || !xq || count < 1 || count > kMaxJobs)
    return fail(QMM_ERR_INVALID, "need 1..%d weights with outputs and an activation", kMaxJobs);
  GemvTarget tg[kMaxJobs];
  for (int j = 0; j < count; ++j) {
    QMM_TRY(check_matmul(w[j], m, y[j], ldy[j]));
    if (!same_act(w[j], w[0])) return fail(QMM_ERR_INVALID, "weights of one launch must share k and dtype (or be Q4_K/Q6_K)");
    tg[j] = {w[j], y[j], ldy[j]};
  }
  if (m > 8) {  // the GEMM runs one weight at a time
    for (int j = 0; j < count; ++j) QMM_TRY(qmm_matmul_q(w[j], xq, m, y[j], ldy[j], ws, ws_bytes, stream));
    return QMM_OK;
  }
  Device* d;
  QMM_TRY(current_device(&d));
  return gemv(d, tg, count, xq, false, 0, (int)m, nullptr, (hipStream_t)stream);
}

int qmm_silu_mul_matmul(const qmm_qtensor* w, const float* g, const float* u, float* y, int accumulate,
                        void* stream) {
  QMM_TRY(check_matmul(w, 1, y, w ? w->n : 0));
  if (!g || !u) return fail(QMM_ERR_INVALID, "null activation");
  if (w->dtype != QMM_Q4K && w->dtype != QMM_Q6K) return fail(QMM_ERR_UNSUPPORTED, "silu prologue needs a k-quant weight");
  Device* d;
  QMM_TRY(current_device(&d));
  GemvTarget t = {w, y, w->n};
  return gemv(d, &t, 1, g, true, w->k, 1, nullptr, (hipStream_t)stream, u, 0.0f, accumulate ? 1 : 0, true);
}

int qmm_matmul_q_ex(const qmm_qtensor* w, const void* xq, int64_t m, float* y, int64_t ldy, int accumulate,
                    void* ws, size_t ws_bytes, void* stream) {
  QMM_TRY(check_matmul(w, m, y, ldy));
  if (!xq) return fail(QMM_ERR_INVALID, "null activation");
  if (!accumulate) return qmm_matmul_q(w, xq, m, y, ldy, ws, ws_bytes, stream);
  if (m > 8) return fail(QMM_ERR_UNSUPPORTED, "accumulating prequantized matmul is limited to m <= 8");
  Device* d;
  QMM_TRY(current_device(&d));
  GemvTarget t = {w, y, ldy};
  return gemv(d, &t, 1, xq, false, 0, (int)m, nullptr, (hipStream_t)stream, nullptr, 0.0f, 1);
}

// Two weights of one shape over the same activation planes (the feed-forward
// block's gate and up) as one unsplit launch of the split-scale tile
// (qmm_mmqs2_q4k, grid z = weight) when each alone would be split over K (a
// grid under half the CUs: 8B gate / up at up to 128 rows) and the pair's
// rounds x K steps are no more than the two split launches': no partials to
// write and read back, one launch fewer (127 rows: 108.9 us for the block
// against 114.4). Unsplit grids stay two launches (512 rows: 349 us against
// 363 paired). QMM_FFN_SEPARATE (or a split count forced by QMM_SPLITK) keeps
// two launches.
static bool pair_plan(const Device* d, const qmm_qtensor* a, const qmm_qtensor* b, int64_t m) {
  // QMM_SPLITK (a forced split count) keeps every weight on its own launch
  if (!use_gemm(a, m) || a->dtype != b->dtype || a->n != b->n || a->k != b->k || env(kEnvFfnPair) != nullptr ||
      env(kEnvSplitK) != nullptr)
    return false;
  const GemmPlan pa = gemm_plan(d, a, m, false);
  if (pa.sk_tiles != 0 || pa.splits < 2 || strcmp(pa.name, "qmm_mmqs_q4k") != 0) return false;
  const long long T = pa.tiles, nbk = a->k / 256, slots = d->num_cu, sp = pa.splits;
  const long long merged = (2 * T + slots - 1) / slots * nbk;
  const long long split = 2 * ((T * sp + slots - 1) / slots) * ((nbk + sp - 1) / sp);
  return merged <= split;
}

static int gemm_pair_launch(Device* d, const qmm_qtensor* a, const qmm_qtensor* b, const uint8_t* planes, int64_t m,
                            float* ya, int64_t lda, float* yb, int64_t ldb, int accumulate, hipStream_t s) {
  if ((uintptr_t)planes % 16) return fail(QMM_ERR_INVALID, "GEMM workspaces must be 16-byte aligned");
  const GemmPlan p = gemm_plan(d, a, m, false);
  const Planes pl = mmq_planes(a->dtype, m, a->k);
  const void* w0 = a->data;
  const void* w1 = b->data;
  const void* q8 = planes + pl.q8;
  const void* dd = planes + pl.d;
  const void* ss = planes + pl.s;
  int M = (int)m, N = (int)a->n, K = (int)a->k, l0 = (int)lda, l1 = (int)ldb, acc = accumulate;
  void* args[] = {&w0, &w1, &q8, &dd, &ss, &ya, &yb, &M, &N, &K, &l0, &l1, &acc};
  hipFunction_t f;
  QMM_TRY(kernel(d, "qmm_mmqs2_q4k", &f));
  QMM_HIP(hipModuleLaunchKernel(f, (unsigned)((N + 127) / 128), (unsigned)((M + 127) / 128), 2, p.threads, 1, 1,
                                p.lds, s, args, nullptr));
  return QMM_OK;
}

// Two or three Q4_K / Q6_K weights of one k over the same activation planes
// (the prefill's q / k / v) as one launch of qmm_mmqs_multi, where each alone
// would be split over K into partials: the split counts are chosen together
// so that every workgroup of the launch fits one round over the CUs (one
// 512-thread workgroup per CU), minimising the longest split (a Q6_K step
// weighted 5 against a Q4_K step's 4), then the partial bytes. The partials
// must fit in the largest of the jobs' own split scratch, so a workspace
// sized for the separate launches holds them. 8B q / k / v at 127 rows:
// splits 4 / 4 / 8 in one launch of 224 workgroups, against 8 / 8 / 8 in
// three. QMM_QKV_SEPARATE (or a split count forced by QMM_SPLITK) keeps one
// launch per weight.
struct MmqsJobs {  // the kernel's by-value argument (qmm_mmqs_multi)
  const void* w[3];
  float* y[3];
  int n[3], gx[3], kc[3], q6[3];
  int start[4];
};
static_assert(sizeof(MmqsJobs) == 112, "qmm_mmqs_multi argument layout");

struct MultiPlan {
  int count = 0, splits[3] = {1, 1, 1}, kc[3] = {0, 0, 0}, gx[3] = {0, 0, 0}, wgs = 0;
  size_t off[3] = {0, 0, 0}, bytes = 0;  // each job's partials in the scratch
};

static bool multi_plan(const Device* d, const qmm_qtensor* const* w, int count, int64_t m, MultiPlan* out) {
  if (count < 2 || count > 3 || env(kEnvQkvSeparate) != nullptr || env(kEnvSplitK) != nullptr) return false;
  size_t bound = 0;
  int q6[3] = {0, 0, 0};
  for (int j = 0; j < count; ++j) {
    if (!w[j] || !use_gemm(w[j], m) || w[j]->k != w[0]->k) return false;
    const int f = fmt_of(w[j]->dtype);
    const GemmPlan pj = gemm_plan(d, w[j], m, false);
    const bool tile = (f == kFmtQ4K && strcmp(pj.name, "qmm_mmqs_q4k") == 0) ||
                      (f == kFmtQ6K && strcmp(pj.name, "qmm_mmqs6_q6k") == 0);
    if (!tile || pj.sk_tiles != 0 || pj.splits < 2) return false;
    q6[j] = f == kFmtQ6K;
    bound = std::max(bound, align256((size_t)pj.splits * (size_t)m * (size_t)w[j]->n * 4));
  }
  const int nbk = (int)(w[0]->k / 256), gy = (int)((m + 127) / 128);
  static const int cand[5] = {1, 2, 4, 8, 16};
  MultiPlan best;
  long long best_path = -1;
  int c[3] = {0, 0, 0};
  const int ncomb = count == 3 ? 125 : 25;
  for (int t = 0; t < ncomb; ++t) {
    c[0] = t % 5;
    c[1] = (t / 5) % 5;
    c[2] = t / 25;
    MultiPlan p;
    p.count = count;
    long long path = 0;
    bool ok = true;
    for (int j = 0; j < count && ok; ++j) {
      const int sp = cand[c[j]];
      const int kc = (nbk + sp - 1) / sp;
      if (sp > nbk || (sp > 1 && kc < 2)) ok = false;
      p.kc[j] = kc;
      p.splits[j] = (nbk + kc - 1) / kc;
      p.gx[j] = (int)((w[j]->n + 127) / 128);
      p.wgs += p.gx[j] * gy * p.splits[j];
      path = std::max(path, (long long)kc * (q6[j] ? 5 : 4));
      p.off[j] = p.bytes;
      p.bytes += align256((size_t)p.splits[j] * (size_t)m * (size_t)w[j]->n * 4);
    }
    if (!ok || p.wgs > d->num_cu || p.bytes > bound) continue;
    if (best_path < 0 || path < best_path || (path == best_path && p.bytes < best.bytes)) {
      best = p;
      best_path = path;
    }
  }
  if (best_path < 0) return false;
  *out = best;
  return true;
}

// The multi launch of plan p over the planes at `planes`: job j's partials at
// part + p.off[j] (split s at + s * m * n_j floats).
static int multi_launch(Device* d, const qmm_qtensor* const* w, const MultiPlan& p, const uint8_t* planes, int64_t m,
                        uint8_t* part, hipStream_t s) {
  if ((uintptr_t)planes % 16) return fail(QMM_ERR_INVALID, "GEMM workspaces must be 16-byte aligned");
  MmqsJobs jobs = {};
  const int gy = (int)((m + 127) / 128);
  int start = 0;
  for (int j = 0; j < 3; ++j) {
    const int jj = j < p.count ? j : p.count - 1;  // unused slots repeat the last job (never selected)
    jobs.w[j] = w[jj]->data;
    jobs.y[j] = (float*)(part + p.off[jj]);
    jobs.n[j] = (int)w[jj]->n;
    jobs.gx[j] = p.gx[jj];
    jobs.kc[j] = p.kc[jj];
    jobs.q6[j] = fmt_of(w[jj]->dtype) == kFmtQ6K;
    jobs.start[j] = start;
    if (j < p.count) start += p.gx[j] * gy * p.splits[j];
  }
  jobs.start[3] = start;
  const Planes pl = mmq_planes(w[0]->dtype, m, w[0]->k);
  const void* q8 = planes + pl.q8;
  const void* dd = planes + pl.d;
  const void* ss = planes + pl.s;
  int M = (int)m, K = (int)w[0]->k;
  void* args[] = {&jobs, &q8, &dd, &ss, &M, &K};
  // the larger of the two tiles' LDS (mmqs: 2 x 72.5 KB, mmqs6: 2 x 71 KB)
  const unsigned lds = 2 * std::max(kS6StageBytes, kSStageBytes);
  return launch(d, "qmm_mmqs_multi", (unsigned)start, 512, lds, s, args);
}

// Shared by qmm_matmul / qmm_matmul_multi: x f32 [m, k] against `count` weights.
static int matmul_targets(const GemvTarget* tg, int count, const float* x, int64_t m, int64_t ldx, void* ws,
                          size_t ws_bytes, void* stream, const float* norm_w = nullptr, float eps = 0.0f,
                          int accumulate = 0) {
  const qmm_qtensor* w = tg[0].w;
  if (!x) return fail(QMM_ERR_INVALID, "null activation");
  if (ldx < w->k) return fail(QMM_ERR_INVALID, "row stride %lld < k %lld", (long long)ldx, (long long)w->k);
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  if (m <= 2) {
    // one launch: the activation is (normalised and) quantized in the GEMV prologue
    return gemv(d, tg, count, x, true, ldx, (int)m, nullptr, s, norm_w, eps, accumulate);
  }
  size_t need = qmm_matmul_workspace_size(w, m);
  const size_t nrm = norm_w ? align256((size_t)(m * w->k) * 4) : 0;
  need += nrm;
  if (!ws || ws_bytes < need) return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, need);
  // layout: quantized activation (GGML rows or GEMM planes), normalised rows,
  // then (GEMM) split-K partials in the rest
  const size_t base = use_gemm(w, m) ? mmq_planes(w->dtype, m, w->k).total : qmm_matmul_workspace_size(w, m);
  // GEMM over Q8_K planes with RMSNorm: one launch normalises each row and
  // writes the planes (the same values as qmm_rms_norm, then the quantizer)
  const bool norm_planes = norm_w && use_gemm(w, m) && qmm_vec_dot_type(w->dtype) == QMM_Q8K &&
                           w->k * 4 <= d->max_lds;
  if (norm_w && !norm_planes) {
    float* xn = (float*)((uint8_t*)ws + base);
    QMM_TRY(qmm_rms_norm(x, m, w->k, ldx, norm_w, eps, xn, w->k, stream));
    x = xn;
    ldx = w->k;
  }
  if (use_gemm(w, m)) {
    if (norm_planes) {
      const Planes pl = mmq_planes(w->dtype, m, w->k);
      long long lx = ldx;
      int kk = (int)w->k;
      void* q8 = (uint8_t*)ws + pl.q8;
      void* dd = (uint8_t*)ws + pl.d;
      void* ss = (uint8_t*)ws + pl.s;
      void* args[] = {&x, &lx, &norm_w, &eps, &kk, &q8, &dd, &ss};
      QMM_TRY(launch(d, "qmm_rms_norm_q8k_mmq", (unsigned)m, 1024, (unsigned)(w->k * 4), s, args));
    } else {
      QMM_TRY(quantize_planes(d, w->dtype, x, m, w->k, ldx, (uint8_t*)ws, s));
    }
    // a job whose split plan needs more than the rest of the workspace runs
    // unsplit (size ws for the largest weight to split every job)
    float* part = (float*)((uint8_t*)ws + base + nrm);
    const size_t sb = ws_bytes - base - nrm;
    if (count == 2 && pair_plan(d, tg[0].w, tg[1].w, m))
      return gemm_pair_launch(d, tg[0].w, tg[1].w, (const uint8_t*)ws, m, tg[0].y, tg[0].ldy, tg[1].y, tg[1].ldy,
                              accumulate, s);
    const qmm_qtensor* wl[3] = {tg[0].w, count > 1 ? tg[1].w : nullptr, count > 2 ? tg[2].w : nullptr};
    MultiPlan mp;
    if (multi_plan(d, wl, count, m, &mp) && mp.bytes <= sb) {
      QMM_TRY(multi_launch(d, wl, mp, (const uint8_t*)ws, m, (uint8_t*)part, s));
      for (int j = 0; j < count; ++j) {
        int M = (int)m, N = (int)tg[j].w->n, sp = mp.splits[j], lo = (int)tg[j].ldy, acc = accumulate;
        const float* pp = (const float*)((uint8_t*)part + mp.off[j]);
        float* yy = tg[j].y;
        void* a2[] = {&pp, &sp, &M, &N, &yy, &lo, &acc};
        QMM_TRY(launch(d, "qmm_splitk_sum", ceil_div((int64_t)M * N, 256), 256, 0, s, a2));
      }
      return QMM_OK;
    }
    for (int j = 0; j < count; ++j)
      QMM_TRY(gemm(d, tg[j].w, (const uint8_t*)ws, m, tg[j].y, tg[j].ldy, nullptr, s, accumulate, part, sb));
    return QMM_OK;
  }
  const int vt = qmm_vec_dot_type(w->dtype);
  QMM_TRY(qmm_quantize_rows(vt, x, m, w->k, ldx, ws, stream));
  const size_t xrow = (size_t)(w->k / qmm_block_size(vt)) * qmm_type_size(vt);
  for (int64_t m0 = 0; m0 < m; m0 += 8) {
    const int mm = (int)(m - m0 < 8 ? m - m0 : 8);
    GemvTarget t[kMaxJobs];
    for (int j = 0; j < count; ++j) t[j] = {tg[j].w, tg[j].y + m0 * tg[j].ldy, tg[j].ldy};
    QMM_TRY(gemv(d, t, count, (const uint8_t*)ws + m0 * xrow, false, 0, mm, nullptr, s, nullptr, 0.0f, accumulate));
  }
  return QMM_OK;
}

int qmm_matmul(const qmm_qtensor* w, const float* x, int64_t m, int64_t ldx, float* y, int64_t ldy, void* ws,
               size_t ws_bytes, void* stream) {
  QMM_TRY(check_matmul(w, m, y, ldy));
  GemvTarget t = {w, y, ldy};
  return matmul_targets(&t, 1, x, m, ldx, ws, ws_bytes, stream);
}

int qmm_matmul_multi(const qmm_qtensor* const* w, int count, const float* x, int64_t m, int64_t ldx,
                     float* const* y, const int64_t* ldy, void* ws, size_t ws_bytes, void* stream) {
  if (!w || !y || !ldy || count < 1 || count > kMaxJobs)
    return fail(QMM_ERR_INVALID, "need 1..%d weights with outputs", kMaxJobs);
  GemvTarget t[kMaxJobs];
  for (int j = 0; j < count; ++j) {
    QMM_TRY(check_matmul(w[j], m, y[j], ldy[j]));
    if (w[j]->dtype != w[0]->dtype || w[j]->k != w[0]->k)
      return fail(QMM_ERR_INVALID, "weights of one multi-matmul must share dtype and k");
    t[j] = {w[j], y[j], ldy[j]};
  }
  return matmul_targets(t, count, x, m, ldx, ws, ws_bytes, stream);
}

// Two groups of one-row GEMVs in one launch (qmm_gemv1g_*): one 16-wave
// workgroup per CU, split between the groups so that the largest per-wave
// share of weight bytes is smallest (rows are dealt to a group's waves as in
// gemv1: a wave of a group of G workgroups takes ceil(rows / (16 G)) rows at
// most). At the config-2 set (q/k/v/gate/up 34816 rows of 2304 B, down 4096
// rows of 8064 B) that is 170 / 86 workgroups: at most 29,952 B per wave
// against 27,700 B for a perfect split.
int qmm_matmul_grouped(const qmm_qtensor* const* w, const int* group, int count, const float* const* x,
                       float* const* y, void* stream) {
  if (!w || !group || !x || !y || count < 1 || count > 16) return fail(QMM_ERR_INVALID, "1..16 weights with groups");
  int njobs[2] = {0, 0};
  long long total[2] = {0, 0};
  int64_t kg[2] = {0, 0};
  const int dtype = w[0] ? w[0]->dtype : -1;
  const int fmt = fmt_of(dtype);
  if (fmt != kFmtQ4K && fmt != kFmtQ6K) return fail(QMM_ERR_UNSUPPORTED, "grouped GEMV: Q4_K or Q6_K weights");
  GemvJobs jobs[2] = {};
  for (int i = 0; i < count; ++i) {
    const int gi = group[i];
    if (!w[i] || !y[i] || (gi != 0 && gi != 1)) return fail(QMM_ERR_INVALID, "weight %d: null, or group not 0/1", i);
    if (w[i]->dtype != dtype) return fail(QMM_ERR_INVALID, "grouped GEMV weights share one dtype");
    if (kg[gi] == 0) kg[gi] = w[i]->k;
    if (w[i]->k != kg[gi]) return fail(QMM_ERR_INVALID, "weights of one group share k");
    if (njobs[gi] == kMaxJobs) return fail(QMM_ERR_INVALID, "at most %d weights per group", kMaxJobs);
    const int j = njobs[gi]++;
    jobs[gi].wq[j] = w[i]->data;
    jobs[gi].y[j] = y[i];
    jobs[gi].rows[j] = (int)w[i]->n;
    jobs[gi].ldy[j] = (int)w[i]->n;
    jobs[gi].row0[j] = 0;
    jobs[gi].trows[j] = (int)w[i]->n;
    total[gi] += w[i]->n;
  }
  for (int gi = 0; gi < 2; ++gi) {
    if (njobs[gi] == 0) continue;
    if (!x[gi]) return fail(QMM_ERR_INVALID, "null activation of group %d", gi);
    if (total[gi] > (1LL << 31) - 1) return fail(QMM_ERR_INVALID, "too many rows in group %d", gi);
    if (kg[gi] / 256 > 64) return fail(QMM_ERR_UNSUPPORTED, "grouped GEMV: k <= 16384");
    jobs[gi].njobs = njobs[gi];
    jobs[gi].total = (int)total[gi];
  }
  Device* d;
  QMM_TRY(current_device(&d));
  const unsigned lds = (unsigned)(std::max(kg[0], kg[1]) / 256 * 292);
  if ((int)lds > d->max_lds) return fail(QMM_ERR_UNSUPPORTED, "activation needs %u B of LDS", lds);
  int G = d->num_cu;
  if (const char* e = env(kEnvGroupedWgs)) G = std::max(2, std::min(8, atoi(e))) * d->num_cu;
  int ga = njobs[1] == 0 ? G : 0;
  if (njobs[0] > 0 && njobs[1] > 0) {
    const long long body = fmt == kFmtQ4K ? 144 : 208;
    long long best = -1;
    for (int a = 1; a < G; ++a) {
      const long long ca = (total[0] + 16LL * a - 1) / (16LL * a) * (kg[0] / 256) * body;
      const long long cb = (total[1] + 16LL * (G - a) - 1) / (16LL * (G - a)) * (kg[1] / 256) * body;
      const long long c = std::max(ca, cb);
      if (best < 0 || c < best) {
        best = c;
        ga = a;
      }
    }
  }
  const float* xa = x[0];
  const float* xb = x[1];
  int ka = (int)kg[0], kb = (int)kg[1], acc = 0;
  void* args[16 * 6 + 10];
  int na = 0;
  for (int gi = 0; gi < 2; ++gi)
    for (int j = 0; j < kMaxJobs; ++j) {
      args[na++] = &jobs[gi].wq[j];
      args[na++] = &jobs[gi].y[j];
      args[na++] = &jobs[gi].rows[j];
      args[na++] = &jobs[gi].ldy[j];
      args[na++] = &jobs[gi].row0[j];
      args[na++] = &jobs[gi].trows[j];
    }
  args[na++] = &jobs[0].njobs;
  args[na++] = &jobs[0].total;
  args[na++] = &jobs[1].njobs;
  args[na++] = &jobs[1].total;
  args[na++] = &xa;
  args[na++] = &xb;
  args[na++] = &ka;
  args[na++] = &kb;
  args[na++] = &ga;
  args[na++] = &acc;
  // a group of rows longer than one wave-wide slice (16 blocks) takes the
  // prefetch ring for its rows (gemv1 would pay a round trip per slice);
  // QMM_GROUPED_P="PA,PB" picks the depths (0: gemv1; instantiated: q4k 0/2,
  // 0/4, 1/4, q6k 0/2, 0/3, and 0/0)
  int pa = 0, pb = 0;
  if (kg[1] / 256 > 16) pb = fmt == kFmtQ4K ? 4 : 2;
  if (kg[0] / 256 > 16 && pb > 0) pa = fmt == kFmtQ4K ? 1 : 0;
  if (const char* e = env(kEnvGroupedP)) {
    if (sscanf(e, "%d,%d", &pa, &pb) != 2) pa = pb = 0;
  }
  char name[48];
  if (pa == 0 && pb == 0)
    snprintf(name, sizeof(name), "qmm_gemv1g_%s_w16", fmt_name(fmt));
  else
    snprintf(name, sizeof(name), "qmm_gemv1g_%s_w16_p%d_p%d", fmt_name(fmt), pa, pb);
  return launch(d, name, (unsigned)G, 1024, lds, (hipStream_t)stream, args);
}

int qmm_matmul_ex(const qmm_qtensor* const* w, int count, const float* x, int64_t m, int64_t ldx,
                  const float* norm_weight, float eps, int accumulate, float* const* y, const int64_t* ldy, void* ws,
                  size_t ws_bytes, void* stream) {
  if (!w || !y || !ldy || count < 1 || count > kMaxJobs)
    return fail(QMM_ERR_INVALID, "need 1..%d weights with outputs", kMaxJobs);
  GemvTarget t[kMaxJobs];
  for (int j = 0; j < count; ++j) {
    QMM_TRY(check_matmul(w[j], m, y[j], ldy[j]));
    if (!same_act(w[j], w[0])) return fail(QMM_ERR_INVALID, "weights of one call must share k and dtype (or be Q4_K/Q6_K)");
    t[j] = {w[j], y[j], ldy[j]};
  }
  // Q4_K and Q6_K jobs share one RMSNorm and one Q8_K quantization: both take
  // Q8_K activations, in the same GGML rows (m <= 8) or GEMM planes (m > 8);
  // each job's GEMV / GEMM then runs its own format (a q/k/v call with a
  // Q6_K v normalised and quantized twice before: 2 x 9.7 us per prefill layer)
  return matmul_targets(t, count, x, m, ldx, ws, ws_bytes, stream, norm_weight, eps, accumulate ? 1 : 0);
}

size_t qmm_matmul_ex_workspace_size(const qmm_qtensor* w, int64_t m, int normalize) {
  if (!w || m <= 0) return 0;
  size_t b = qmm_matmul_workspace_size(w, m);
  if (normalize && m > 2) b += align256((size_t)(m * w->k) * 4);
  return b;
}

// ---------------------------------------------------------------------------
// the feed-forward block of a prompt's rows: y (+)= down(silu(gate(n)) * up(n))
// ---------------------------------------------------------------------------

// The GEMM planes of m input rows at `xp` (Q8_K layout of dtype `wdtype`),
// RMS-normalised first when norm_weight is given: one launch when a row fits
// in LDS, else qmm_rms_norm into `xn` (m x k floats) and the quantizer.
static int input_planes(Device* d, int wdtype, const float* x, int64_t m, int64_t k, int64_t ldx,
                        const float* norm_weight, float eps, uint8_t* xp, float* xn, hipStream_t s) {
  const Planes px = mmq_planes(wdtype, m, k);
  if (norm_weight && (size_t)k * 4 <= (size_t)d->max_lds) {
    long long lx = ldx;
    int kk = (int)k;
    void* q8 = xp + px.q8;
    void* dd = xp + px.d;
    void* ss = xp + px.s;
    void* args[] = {&x, &lx, &norm_weight, &eps, &kk, &q8, &dd, &ss};
    return launch(d, "qmm_rms_norm_q8k_mmq", (unsigned)m, 1024, (unsigned)(k * 4), s, args);
  }
  const float* xs = x;
  int64_t lx = ldx;
  if (norm_weight) {
    QMM_TRY(qmm_rms_norm(x, m, k, ldx, norm_weight, eps, xn, k, s));
    xs = xn;
    lx = k;
  }
  return quantize_planes(d, wdtype, xs, m, k, lx, xp, s);
}

// Workspace regions of qmm_ffn. m > 8 (GEMMs): the input's planes (and its
// normalised rows when the fused norm-planes launch cannot hold a row in LDS),
// gate's and up's outputs as their split-K partials (one plane when a GEMM
// runs unsplit), the SiLU product's planes, the down GEMM's split partials.
// m <= 8 (GEMVs): gate / up outputs, the product's Q8_K rows, then
// qmm_matmul_ex's workspace for gate / up.
struct FfnWs {
  size_t xp, xn, g, u, hp, part, total;
  int gsplits, usplits;
};

static int ffn_check(const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, int64_t m) {
  if (!gate || !up || !down) return fail(QMM_ERR_INVALID, "null weight");
  if (m < 1) return fail(QMM_ERR_INVALID, "ffn needs m >= 1 (got %lld)", (long long)m);
  if (qmm_vec_dot_type(gate->dtype) != QMM_Q8K || qmm_vec_dot_type(down->dtype) != QMM_Q8K || !same_act(gate, up))
    return fail(QMM_ERR_UNSUPPORTED, "ffn needs Q4_K / Q6_K gate, up and down weights");
  if (gate->n != up->n || down->k != gate->n)
    return fail(QMM_ERR_INVALID, "ffn shapes: gate %lldx%lld, up %lldx%lld, down %lldx%lld", (long long)gate->n,
                (long long)gate->k, (long long)up->n, (long long)up->k, (long long)down->n, (long long)down->k);
  return QMM_OK;
}

static FfnWs ffn_ws(Device* d, const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, int64_t m,
                    bool normalize) {
  FfnWs w = {};
  const int64_t H = gate->k, F = gate->n;
  size_t o = 0;
  if (m > 8) {
    w.xp = o;
    o += mmq_planes(gate->dtype, m, H).total;
    w.xn = o;
    if (normalize && (size_t)H * 4 > (size_t)d->max_lds) o += align256((size_t)(m * H) * 4);
    w.gsplits = gemm_plan(d, gate, m, false).splits;
    w.usplits = gemm_plan(d, up, m, false).splits;
    w.g = o;
    o += align256((size_t)w.gsplits * (size_t)(m * F) * 4);
    w.u = o;
    o += align256((size_t)w.usplits * (size_t)(m * F) * 4);
    w.hp = o;
    o += mmq_planes(down->dtype, m, F).total;
    w.part = o;  // down's split partials or stream-K scratch, and gate's / up's stream-K scratch
    o += std::max(gemm_split_bytes(down, m), std::max(gemm_sk_bytes(d, gate, m), gemm_sk_bytes(d, up, m)));
  } else {
    w.g = o;
    o += align256((size_t)(m * F) * 4);
    w.u = o;
    o += align256((size_t)(m * F) * 4);
    w.hp = o;
    o += align256((size_t)m * (size_t)(F / 256) * (size_t)qmm_type_size(QMM_Q8K));
    w.part = o;
    o += std::max(qmm_matmul_ex_workspace_size(gate, m, normalize ? 1 : 0),
                  qmm_matmul_ex_workspace_size(up, m, normalize ? 1 : 0));
  }
  w.total = o;
  return w;
}

size_t qmm_ffn_workspace_size(const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, int64_t m,
                              int normalize) {
  if (ffn_check(gate, up, down, m) != QMM_OK) return 0;
  Device* d;
  if (current_device(&d) != QMM_OK) return 0;
  return ffn_ws(d, gate, up, down, m, normalize != 0).total;
}

int qmm_ffn(const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, const float* x, int64_t m,
            int64_t ldx, const float* norm_weight, float eps, int accumulate, float* y, int64_t ldy, void* ws,
            size_t ws_bytes, void* stream) {
  QMM_TRY(ffn_check(gate, up, down, m));
  QMM_TRY(check_matmul(down, m, y, ldy));
  if (!x) return fail(QMM_ERR_INVALID, "null activation");
  const int64_t H = gate->k, F = gate->n;
  if (ldx < H) return fail(QMM_ERR_INVALID, "row stride %lld < k %lld", (long long)ldx, (long long)H);
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  const FfnWs L = ffn_ws(d, gate, up, down, m, norm_weight != nullptr);
  if (!ws || ws_bytes < L.total) return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, L.total);
  uint8_t* b = (uint8_t*)ws;
  float* g = (float*)(b + L.g);
  float* u = (float*)(b + L.u);
  if (m <= 8) {
    const qmm_qtensor* gw[2] = {gate, up};
    float* gy[2] = {g, u};
    const int64_t ld2[2] = {F, F};
    QMM_TRY(qmm_matmul_ex(gw, 2, x, m, ldx, norm_weight, eps, 0, gy, ld2, b + L.part, ws_bytes - L.part, stream));
    QMM_TRY(qmm_silu_mul_quantize(g, u, m, F, F, b + L.hp, stream));
    return qmm_matmul_q_ex(down, b + L.hp, m, y, ldy, accumulate, nullptr, 0, stream);
  }
  // the input's Q8_K planes, normalised on the way when asked
  QMM_TRY(input_planes(d, gate->dtype, x, m, H, ldx, norm_weight, eps, b + L.xp, (float*)(b + L.xn), s));
  // gate and up: one launch over both when pair_plan takes them (unsplit),
  // else their split partials left unsummed
  const GemmPlan pg = gemm_plan(d, gate, m, false), pu = gemm_plan(d, up, m, false);
  const bool pair = pair_plan(d, gate, up, m);
  if (pair) {
    QMM_TRY(gemm_pair_launch(d, gate, up, b + L.xp, m, g, F, u, F, 0, s));
  } else {
    QMM_TRY(gemm_launch(d, gate, b + L.xp, m, pg, g, F, nullptr, s, 0, g, b + L.part));
    QMM_TRY(gemm_launch(d, up, b + L.xp, m, pu, u, F, nullptr, s, 0, u, b + L.part));
  }
  // split sums, silu(g) * u and the down GEMM's Q8_K planes in one launch
  {
    const Planes ph = mmq_planes(down->dtype, m, F);
    const float* gp = g;
    const float* upp = u;
    int gsp = pair ? 1 : pg.splits, usp = pair ? 1 : pu.splits, kk = (int)F, mm = (int)m;
    void* q8 = b + L.hp + ph.q8;
    void* dd = b + L.hp + ph.d;
    void* ss = b + L.hp + ph.s;
    void* args[] = {&gp, &gsp, &upp, &usp, &q8, &dd, &ss, &kk, &mm};
    QMM_TRY(launch(d, "qmm_splitk_silu_mul_q8k_mmq", ceil_div(m * (F / 256), 4), 256, 0, s, args));
  }
  return gemm(d, down, b + L.hp, m, y, ldy, nullptr, s, accumulate, (float*)(b + L.part), ws_bytes - L.part);
}

// ---------------------------------------------------------------------------
// q / k / v of a prompt's rows with RoPE and the KV append
// ---------------------------------------------------------------------------

// Workspace regions: m > 8, the input's planes (and normalised rows), then
// q's, k's and v's split-K partials (one plane each when unsplit); m <= 8,
// the k and v rows, then qmm_matmul_ex's workspace.
struct QkvWs {
  size_t xp, xn, q, k, v, mm, total;
};

// What the weights alone fix (the workspace query has no attention geometry).
static int qkv_check_weights(const qmm_qtensor* wq, const qmm_qtensor* wk, const qmm_qtensor* wv, int64_t m) {
  if (!wq || !wk || !wv) return fail(QMM_ERR_INVALID, "null weight");
  if (m < 1) return fail(QMM_ERR_INVALID, "qkv needs m >= 1 (got %lld)", (long long)m);
  if (qmm_vec_dot_type(wq->dtype) != QMM_Q8K || !same_act(wq, wk) || !same_act(wq, wv))
    return fail(QMM_ERR_UNSUPPORTED, "qkv needs Q4_K / Q6_K weights of one k");
  if (wv->n != wk->n)
    return fail(QMM_ERR_INVALID, "k and v weights of %lld / %lld rows", (long long)wk->n, (long long)wv->n);
  return QMM_OK;
}

static int qkv_check(const qmm_qtensor* wq, const qmm_qtensor* wk, const qmm_qtensor* wv, int64_t m, int heads,
                     int kv_heads, int head_dim) {
  QMM_TRY(qkv_check_weights(wq, wk, wv, m));
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 2 || head_dim > 1024 || head_dim % 2)
    return fail(QMM_ERR_INVALID, "bad attention geometry");
  if (wq->n != (int64_t)heads * head_dim || wk->n != (int64_t)kv_heads * head_dim || wv->n != wk->n)
    return fail(QMM_ERR_INVALID, "qkv weights of %lld / %lld / %lld rows for %d x %d / %d x %d heads",
                (long long)wq->n, (long long)wk->n, (long long)wv->n, heads, head_dim, kv_heads, head_dim);
  return QMM_OK;
}

static QkvWs qkv_ws(Device* d, const qmm_qtensor* wq, const qmm_qtensor* wk, const qmm_qtensor* wv, int64_t m,
                    bool normalize) {
  QkvWs w = {};
  const int64_t H = wq->k;
  size_t o = 0;
  if (m > 8) {
    w.xp = o;
    o += mmq_planes(wq->dtype, m, H).total;
    w.xn = o;
    if (normalize && (size_t)H * 4 > (size_t)d->max_lds) o += align256((size_t)(m * H) * 4);
    const qmm_qtensor* ws3[3] = {wq, wk, wv};
    size_t* at[3] = {&w.q, &w.k, &w.v};
    MultiPlan mp;
    const bool multi = multi_plan(d, ws3, 3, m, &mp);
    for (int j = 0; j < 3; ++j) {
      *at[j] = o;
      const int sp = multi ? mp.splits[j] : gemm_plan(d, ws3[j], m, false).splits;
      o += align256((size_t)sp * (size_t)(m * ws3[j]->n) * 4);
    }
    w.mm = o;  // the stream-K scratch of q's, k's and v's GEMMs (one at a time)
    o += std::max(gemm_sk_bytes(d, wq, m), std::max(gemm_sk_bytes(d, wk, m), gemm_sk_bytes(d, wv, m)));
  } else {
    w.k = o;
    o += align256((size_t)(m * wk->n) * 4);
    w.v = o;
    o += align256((size_t)(m * wv->n) * 4);
    w.mm = o;
    o += std::max(qmm_matmul_ex_workspace_size(wq, m, normalize ? 1 : 0),
                  std::max(qmm_matmul_ex_workspace_size(wk, m, normalize ? 1 : 0),
                           qmm_matmul_ex_workspace_size(wv, m, normalize ? 1 : 0)));
  }
  w.total = o;
  return w;
}

size_t qmm_qkv_rope_kv_append_n_workspace_size(const qmm_qtensor* wq, const qmm_qtensor* wk, const qmm_qtensor* wv,
                                               int64_t m, int normalize) {
  if (qkv_check_weights(wq, wk, wv, m) != QMM_OK) return 0;
  Device* d;
  if (current_device(&d) != QMM_OK) return 0;
  return qkv_ws(d, wq, wk, wv, m, normalize != 0).total;
}

int qmm_qkv_rope_kv_append_n(const qmm_qtensor* wq, const qmm_qtensor* wk, const qmm_qtensor* wv, const float* x,
                             int64_t m, int64_t ldx, const float* norm_weight, float eps, const float* cos_t,
                             const float* sin_t, int64_t first, float* q, int64_t ldq, float* kcache,
                             float* vcache, int heads, int kv_heads, int head_dim, int max_seq, void* ws,
                             size_t ws_bytes, void* stream) {
  QMM_TRY(qkv_check(wq, wk, wv, m, heads, kv_heads, head_dim));
  if (!x || !q || !cos_t || !sin_t || !kcache || !vcache) return fail(QMM_ERR_INVALID, "null pointer");
  const int64_t H = wq->k, nq = wq->n, nkv = wk->n;
  if (ldx < H || ldq < nq) return fail(QMM_ERR_INVALID, "row strides below the row widths");
  if (max_seq < 1 || first < 0 || first + m > max_seq || m > 65535)
    return fail(QMM_ERR_INVALID, "positions [%lld, %lld) outside the cache of %d", (long long)first,
                (long long)(first + m), max_seq);
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  const QkvWs L = qkv_ws(d, wq, wk, wv, m, norm_weight != nullptr);
  if (!ws || ws_bytes < L.total) return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, L.total);
  uint8_t* b = (uint8_t*)ws;
  if (m <= 8) {
    float* k = (float*)(b + L.k);
    float* v = (float*)(b + L.v);
    const qmm_qtensor* w3[3] = {wq, wk, wv};
    float* y3[3] = {q, k, v};
    const int64_t ld3[3] = {ldq, nkv, nkv};
    QMM_TRY(qmm_matmul_ex(w3, 3, x, m, ldx, norm_weight, eps, 0, y3, ld3, b + L.mm, ws_bytes - L.mm, stream));
    return qmm_rope_kv_append_n(q, k, v, ldq, nkv, nkv, cos_t, sin_t, first, m, kcache, vcache, heads, kv_heads,
                                head_dim, max_seq, stream);
  }
  QMM_TRY(input_planes(d, wq->dtype, x, m, H, ldx, norm_weight, eps, b + L.xp, (float*)(b + L.xn), s));
  const qmm_qtensor* w3[3] = {wq, wk, wv};
  float* p3[3] = {(float*)(b + L.q), (float*)(b + L.k), (float*)(b + L.v)};
  int sp[3];
  MultiPlan mp;
  if (multi_plan(d, w3, 3, m, &mp)) {
    // one launch over the three weights; its partials in the q / k / v regions (consecutive, in that order)
    for (int j = 0; j < 3; ++j) {
      sp[j] = mp.splits[j];
      mp.off[j] = (size_t)((uint8_t*)p3[j] - (b + L.q));
    }
    QMM_TRY(multi_launch(d, w3, mp, b + L.xp, m, b + L.q, s));
  } else {
    for (int j = 0; j < 3; ++j) {
      const GemmPlan pj = gemm_plan(d, w3[j], m, false);
      sp[j] = pj.splits;
      QMM_TRY(gemm_launch(d, w3[j], b + L.xp, m, pj, p3[j], w3[j]->n, nullptr, s, 0, p3[j], b + L.mm));
    }
  }
  const float* qp = p3[0];
  const float* kp = p3[1];
  const float* vp = p3[2];
  int mm = (int)m, f = (int)first;
  long long lq = ldq;
  void* args[] = {&qp, &sp[0], &kp, &sp[1], &vp, &sp[2], &mm, &q, &lq, &cos_t, &sin_t, &f, &kcache, &vcache,
                  &heads, &kv_heads, &head_dim, &max_seq};
  const unsigned threads = (unsigned)((head_dim + 63) / 64 * 64);
  hipFunction_t fn;
  QMM_TRY(kernel(d, "qmm_prefill_splitk_rope_kv", &fn));
  QMM_HIP(hipModuleLaunchKernel(fn, (unsigned)(heads + kv_heads), (unsigned)m, 1, threads, 1, 1, 0, s, args,
                                nullptr));
  return QMM_OK;
}

// ---------------------------------------------------------------------------
// decode-step kernels (f32, non-matmul)
// ---------------------------------------------------------------------------

int qmm_rms_norm(const float* x, int64_t m, int64_t k, int64_t ldx, const float* w, float eps, float* out,
                 int64_t ldo, void* stream) {
  if (!x || !w || !out || m < 1 || k < 1 || ldx < k || ldo < k) return fail(QMM_ERR_INVALID, "bad rms_norm arguments");
  Device* d;
  QMM_TRY(current_device(&d));
  long long lx = ldx, lo = ldo;
  int kk = (int)k;
  void* args[] = {&x, &lx, &w, &eps, &kk, &out, &lo};
  return launch(d, "qmm_rms_norm", (unsigned)m, 256, 0, (hipStream_t)stream, args);
}

int qmm_embed_rows(const float* table, int64_t ld, int64_t vocab, const int32_t* tokens, const int32_t* pos, float* x,
                   int64_t hidden, void* stream) {
  if (!table || !tokens || !pos || !x || hidden < 1 || ld < hidden || vocab < 1 || vocab > (1LL << 31) - 1)
    return fail(QMM_ERR_INVALID, "bad embed arguments");
  Device* d;
  QMM_TRY(current_device(&d));
  long long l = ld;
  int h = (int)hidden, v = (int)vocab;
  void* args[] = {&table, &l, &v, &tokens, &pos, &x, &h};
  return launch(d, "qmm_decode_embed", ceil_div(hidden, 256), 256, 0, (hipStream_t)stream, args);
}

int qmm_rope_kv_append(float* q, float* k, const float* v, const float* cos_t, const float* sin_t,
                       const int32_t* pos, float* kcache, float* vcache, int heads, int kv_heads, int head_dim,
                       int max_seq, void* stream) {
  if (!q || !k || !v || !cos_t || !sin_t || !pos || !kcache || !vcache) return fail(QMM_ERR_INVALID, "null pointer");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 2 || head_dim > 1024 || head_dim % 2 || max_seq < 1)
    return fail(QMM_ERR_INVALID, "bad attention geometry");
  Device* d;
  QMM_TRY(current_device(&d));
  void* args[] = {&q, &k, &v, &cos_t, &sin_t, &pos, &kcache, &vcache, &heads, &kv_heads, &head_dim, &max_seq};
  const unsigned threads = (unsigned)((head_dim + 63) / 64 * 64);
  return launch(d, "qmm_decode_rope_kv", (unsigned)(heads + kv_heads), threads, 0, (hipStream_t)stream, args);
}

// Workspace of the attention: one counter per kv head (a 256-byte-aligned
// region), then S chunks x heads x (m, l, o[head_dim]) floats.
static const int kAttnSplits = 16;  // must equal the kernel's qmm::kAttnSplits
// Positions per cache: the kernels index positions with 32-bit integers and
// the cache with 64-bit offsets; 2^20 keeps every position count, and each
// chunk's scan, far inside that.
static const int kAttnMaxSeq = 1 << 20;


static int check_attention(int heads, int kv_heads, int head_dim, int max_seq) {
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || heads / kv_heads > 8)
    return fail(QMM_ERR_INVALID, "attention needs heads %% kv_heads == 0 and heads / kv_heads <= 8");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(QMM_ERR_INVALID, "attention head_dim must be 64, 128 or 256 (got %d)", head_dim);
  if (max_seq < 1 || max_seq > kAttnMaxSeq)
    return fail(QMM_ERR_INVALID, "attention max_seq must be in [1, %d] (got %d)", kAttnMaxSeq, max_seq);
  return QMM_OK;
}

static size_t attn_counter_bytes(int kv_heads) { return ((size_t)kv_heads * 4 + 255) / 256 * 256; }

// L2 warming by the attention launch (see qmm_decode_kernels.h): the weights of
// the one-row GEMV launches that follow the attention, each with the launch it
// belongs to (jobs of one launch consecutive, launches in order) and the rows
// per wave of that launch to load. The consuming launches' geometry is the one
// gemv() gives a fused one-row launch: 16-wave workgroups, min(rows / 16, CUs)
// of them.
struct WarmPlan {
  const void* w[3];
  unsigned row_bytes[3];
  int rows[3], first[3], grid_waves[3], kmax[3];
  int njobs = 0;
};
static int warm_plan(const Device* d, const qmm_qtensor* const* warm, const int* warm_launch, int count,
                     const int* warm_rows, WarmPlan* out) {
  WarmPlan p;
  if (count == 0) {
    *out = p;
    return QMM_OK;
  }
  if (!warm || !warm_launch || !warm_rows || count < 0 || count > 3)
    return fail(QMM_ERR_INVALID, "L2 warming takes 0..3 weights with their launches and rows per wave");
  int launch = -1, first = 0;
  long long total = 0;
  int start = 0;
  for (int i = 0; i <= count; ++i) {
    // close the previous launch: every job of it gets the launch's wave count
    if (i == count || (i > 0 && warm_launch[i] != warm_launch[i - 1])) {
      const long long wgs = std::min<long long>((total + 15) / 16, d->num_cu);
      for (int j = start; j < i; ++j) p.grid_waves[j] = (int)(wgs * 16);
      start = i;
      total = 0;
      first = 0;
      if (i == count) break;
    }
    const qmm_qtensor* w = warm[i];
    if (!w || fmt_of(w->dtype) == kFmtQ80) return fail(QMM_ERR_INVALID, "L2 warming takes Q4_K / Q6_K weights");
    if (warm_launch[i] < launch || warm_launch[i] < 0) return fail(QMM_ERR_INVALID, "warm_launch must not decrease");
    launch = warm_launch[i];
    const int rpw = warm_rows[launch];
    if (rpw < 0 || rpw > 64) return fail(QMM_ERR_INVALID, "rows per wave to warm: 0..64");
    p.w[i] = w->data;
    p.row_bytes[i] = (unsigned)((w->k / 256) * (fmt_of(w->dtype) == kFmtQ4K ? 144 : 208));
    p.rows[i] = (int)w->n;
    p.first[i] = first;
    p.kmax[i] = rpw;
    first += (int)w->n;
    total += w->n;
  }
  p.njobs = count;
  *out = p;
  return QMM_OK;
}

size_t qmm_decode_attention_workspace_size(int heads, int kv_heads, int head_dim, int max_seq) {
  if (check_attention(heads, kv_heads, head_dim, max_seq) != QMM_OK) return 0;
  return attn_counter_bytes(kv_heads) + (size_t)kAttnSplits * heads * (head_dim + 2) * sizeof(float);
}

static int attention(const float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                     const int32_t* pos, float* kcache, float* vcache, float* out, int heads, int kv_heads,
                     int head_dim, int max_seq, float scale, void* ws, size_t ws_bytes, void* stream,
                     const qmm_qtensor* const* warm = nullptr, const int* warm_launch = nullptr, int warm_count = 0,
                     const int* warm_rows = nullptr) {
  QMM_TRY(check_attention(heads, kv_heads, head_dim, max_seq));
  const size_t need = qmm_decode_attention_workspace_size(heads, kv_heads, head_dim, max_seq);
  if (!ws || ws_bytes < need) return fail(QMM_ERR_INVALID, "attention workspace of %zu B < %zu B", ws_bytes, need);
  Device* d;
  QMM_TRY(current_device(&d));
  WarmPlan wp;
  QMM_TRY(warm_plan(d, warm, warm_launch, warm_count, warm_rows, &wp));
  unsigned* counters = (unsigned*)ws;
  float* part = (float*)((uint8_t*)ws + attn_counter_bytes(kv_heads));
  const int G = heads / kv_heads;
  const int gt = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
  // eight waves where the kernel's LDS staging of 32 rows fits (gt * head_dim
  // <= 512); config 3 (head_dim 128, G = 4): 508 -> 520 tok/s over four waves
  const int splits = kAttnSplits, nw = gt * head_dim <= 512 ? 8 : 4;
  char name[64];
  snprintf(name, sizeof(name), "qmm_decode_attention_d%d_g%d_w%d", head_dim / 64, gt, nw);
  int pf_nw = 16, pf_njobs = wp.njobs;
  void* args[] = {&q, &k, &v, &cos_t, &sin_t, &pos, &kcache, &vcache, &part, &counters, &out,
                  &heads, &kv_heads, &max_seq, &scale,
                  &wp.w[0], &wp.row_bytes[0], &wp.rows[0], &wp.first[0], &wp.grid_waves[0], &wp.kmax[0],
                  &wp.w[1], &wp.row_bytes[1], &wp.rows[1], &wp.first[1], &wp.grid_waves[1], &wp.kmax[1],
                  &wp.w[2], &wp.row_bytes[2], &wp.rows[2], &wp.first[2], &wp.grid_waves[2], &wp.kmax[2],
                  &pf_njobs, &pf_nw};
  // warming workgroups in grid rows past the attention's (kv_heads * splits of
  // them, a multiple of 8): as many as the CUs the attention leaves free (the
  // kernel's registers hold one of its workgroups per CU), in whole rows of
  // kv_heads and a multiple of 8 in all, so that warming workgroup j and the
  // consuming workgroups j, j + nwarm, ... share an XCD
  int gy = splits;
  if (wp.njobs > 0) {
    int rows_y = std::max(1, (d->num_cu - kv_heads * splits) / kv_heads);
    while (rows_y > 1 && (rows_y * kv_heads) % 8) --rows_y;
    if ((rows_y * kv_heads) % 8 == 0) gy += rows_y;
  }
  hipFunction_t f;
  QMM_TRY(kernel(d, name, &f));
  QMM_HIP(hipModuleLaunchKernel(f, (unsigned)kv_heads, (unsigned)gy, 1, (unsigned)(64 * nw), 1, 1, 0,
                                (hipStream_t)stream, args, nullptr));
  return QMM_OK;
}

int qmm_decode_attention(const float* q, const float* kcache, const float* vcache, const int32_t* pos, float* out,
                         int heads, int kv_heads, int head_dim, int max_seq, float scale, void* ws, size_t ws_bytes,
                         void* stream) {
  if (!q || !kcache || !vcache || !pos || !out) return fail(QMM_ERR_INVALID, "null pointer");
  return attention(q, nullptr, nullptr, nullptr, nullptr, pos, const_cast<float*>(kcache),
                   const_cast<float*>(vcache), out, heads, kv_heads, head_dim, max_seq, scale, ws, ws_bytes, stream);
}

int qmm_decode_rope_attention(const float* q, const float* k, const float* v, const float* cos_t,
                              const float* sin_t, const int32_t* pos, float* kcache, float* vcache, float* out,
                              int heads, int kv_heads, int head_dim, int max_seq, float scale, void* ws,
                              size_t ws_bytes, void* stream) {
  if (!q || !k || !v || !cos_t || !sin_t || !pos || !kcache || !vcache || !out)
    return fail(QMM_ERR_INVALID, "null pointer");
  return attention(q, k, v, cos_t, sin_t, pos, kcache, vcache, out, heads, kv_heads, head_dim, max_seq, scale, ws,
                   ws_bytes, stream);
}

int qmm_decode_rope_attention_warm(const float* q, const float* k, const float* v, const float* cos_t,
                                   const float* sin_t, const int32_t* pos, float* kcache, float* vcache, float* out,
                                   int heads, int kv_heads, int head_dim, int max_seq, float scale, void* ws,
                                   size_t ws_bytes, const qmm_qtensor* const* warm, const int* warm_launch,
                                   int warm_count, const int* warm_rows, void* stream) {
  if (!q || !k || !v || !cos_t || !sin_t || !pos || !kcache || !vcache || !out)
    return fail(QMM_ERR_INVALID, "null pointer");
  return attention(q, k, v, cos_t, sin_t, pos, kcache, vcache, out, heads, kv_heads, head_dim, max_seq, scale, ws,
                   ws_bytes, stream, warm, warm_launch, warm_count, warm_rows);
}

// ---------------------------------------------------------------------------
// batched prefill (the prompt's rows through one pass per layer)
// ---------------------------------------------------------------------------

int qmm_embed_rows_n(const float* table, int64_t ld, int64_t vocab, const int32_t* tokens, int64_t first,
                     int64_t count, float* x, int64_t hidden, void* stream) {
  if (!table || !tokens || !x || hidden < 1 || ld < hidden || first < 0 || count < 0 || count > 65535 ||
      first + count > (1LL << 31) - 1 || vocab < 1 || vocab > (1LL << 31) - 1)
    return fail(QMM_ERR_INVALID, "bad embed arguments");
  if (count == 0) return QMM_OK;
  Device* d;
  QMM_TRY(current_device(&d));
  long long l = ld;
  int h = (int)hidden, f = (int)first, v = (int)vocab;
  void* args[] = {&table, &l, &v, &tokens, &f, &x, &h};
  hipFunction_t fn;
  QMM_TRY(kernel(d, "qmm_prefill_embed", &fn));
  QMM_HIP(hipModuleLaunchKernel(fn, std::min(ceil_div(hidden, 256), 64u), (unsigned)count, 1, 256, 1, 1, 0,
                                (hipStream_t)stream, args, nullptr));
  return QMM_OK;
}

int qmm_rope_kv_append_n(float* q, float* k, const float* v, int64_t ldq, int64_t ldk, int64_t ldv,
                         const float* cos_t, const float* sin_t, int64_t first, int64_t count, float* kcache,
                         float* vcache, int heads, int kv_heads, int head_dim, int max_seq, void* stream) {
  if (!q || !k || !v || !cos_t || !sin_t || !kcache || !vcache) return fail(QMM_ERR_INVALID, "null pointer");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 2 || head_dim > 1024 || head_dim % 2 || max_seq < 1)
    return fail(QMM_ERR_INVALID, "bad attention geometry");
  if (first < 0 || count < 0 || first + count > max_seq || count > 65535)
    return fail(QMM_ERR_INVALID, "positions [%lld, %lld) outside the cache of %d", (long long)first,
                (long long)(first + count), max_seq);
  if (ldq < (int64_t)heads * head_dim || ldk < (int64_t)kv_heads * head_dim || ldv < (int64_t)kv_heads * head_dim)
    return fail(QMM_ERR_INVALID, "row strides below the row widths");
  if (count == 0) return QMM_OK;
  Device* d;
  QMM_TRY(current_device(&d));
  long long a = ldq, b = ldk, c = ldv;
  int f = (int)first;
  void* args[] = {&q, &k, &v, &a, &b, &c, &cos_t, &sin_t, &f, &kcache, &vcache, &heads, &head_dim, &max_seq};
  hipFunction_t fn;
  QMM_TRY(kernel(d, "qmm_prefill_rope_kv", &fn));
  const unsigned threads = (unsigned)((head_dim + 63) / 64 * 64);
  QMM_HIP(hipModuleLaunchKernel(fn, (unsigned)(heads + kv_heads), (unsigned)count, 1, threads, 1, 1, 0,
                                (hipStream_t)stream, args, nullptr));
  return QMM_OK;
}

int qmm_prefill_attention(const float* q, int64_t ldq, const float* kcache, const float* vcache, int64_t first,
                          int64_t count, float* out, int64_t ldo, int heads, int kv_heads, int head_dim, int max_seq,
                          float scale, void* stream) {
  if (!q || !kcache || !vcache || !out) return fail(QMM_ERR_INVALID, "null pointer");
  QMM_TRY(check_attention(heads, kv_heads, head_dim, max_seq));
  if (first < 0 || count < 0 || first + count > max_seq || count > 65535)
    return fail(QMM_ERR_INVALID, "positions [%lld, %lld) outside the cache of %d", (long long)first,
                (long long)(first + count), max_seq);
  if (ldq < (int64_t)heads * head_dim || ldo < (int64_t)heads * head_dim)
    return fail(QMM_ERR_INVALID, "row strides below heads * head_dim");
  if (count == 0) return QMM_OK;
  Device* d;
  QMM_TRY(current_device(&d));
  const int G = heads / kv_heads;
  const int gt = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
  char name[64];
  snprintf(name, sizeof(name), "qmm_prefill_attention_d%d_g%d", head_dim / 64, gt);
  long long a = ldq, o = ldo;
  int f = (int)first;
  void* args[] = {&q, &a, &kcache, &vcache, &f, &out, &o, &heads, &kv_heads, &max_seq, &scale};
  hipFunction_t fn;
  QMM_TRY(kernel(d, name, &fn));
  QMM_HIP(hipModuleLaunchKernel(fn, (unsigned)kv_heads, (unsigned)count, 1, 256, 1, 1, 0, (hipStream_t)stream, args,
                                nullptr));
  return QMM_OK;
}

// Attention of the prompt rows followed by the o projection added into the
// residual (LlamaAttention::forward's o_proj and the decoder layer's residual
// add, llama.rs:1115-1120, 654-725): where the o GEMM takes Q8_K planes
// (m > 8, a k-quant weight) and a kv head's G * head_dim outputs are whole
// 256-element blocks, the attention launch writes the planes itself
// (qmm_prefill_attention_planes_*), so the f32 rows and the plane quantizer's
// launch drop out; the GEMM then runs as qmm_matmul_ex runs it. Otherwise the
// two calls. Either way the bits of qmm_prefill_attention followed by
// qmm_matmul_ex(o, accumulate = 1).
size_t qmm_prefill_attention_o_workspace_size(const qmm_qtensor* wo, int64_t count) {
  if (!wo || count < 1) return 0;
  const size_t mm = qmm_matmul_ex_workspace_size(wo, count, 0);
  if (mm == 0) return 0;
  return align256((size_t)count * (size_t)wo->k * 4) + mm;
}

int qmm_prefill_attention_o(const float* q, int64_t ldq, const float* kcache, const float* vcache, int64_t first,
                            int64_t count, int heads, int kv_heads, int head_dim, int max_seq, float scale,
                            const qmm_qtensor* wo, float* x, int64_t ldx, void* ws, size_t ws_bytes, void* stream) {
  if (!q || !kcache || !vcache || !wo || !x) return fail(QMM_ERR_INVALID, "null pointer");
  QMM_TRY(check_attention(heads, kv_heads, head_dim, max_seq));
  const int64_t H = (int64_t)heads * head_dim;
  if (wo->k != H)
    return fail(QMM_ERR_INVALID, "o weight of k = %lld for %lld attention outputs", (long long)wo->k, (long long)H);
  if (first < 0 || count < 0 || first + count > max_seq || count > 65535)
    return fail(QMM_ERR_INVALID, "positions [%lld, %lld) outside the cache of %d", (long long)first,
                (long long)(first + count), max_seq);
  if (ldq < H || ldx < wo->n) return fail(QMM_ERR_INVALID, "row strides below the row widths");
  if (count == 0) return QMM_OK;
  const size_t need = qmm_prefill_attention_o_workspace_size(wo, count);
  if (need == 0) return fail(QMM_ERR_UNSUPPORTED, "o weight format not supported");
  if (!ws || ws_bytes < need) return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, need);
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* b = (uint8_t*)ws;
  const int G = heads / kv_heads;
  const bool fuse = use_gemm(wo, count) && qmm_vec_dot_type(wo->dtype) == QMM_Q8K && (G * head_dim) % 256 == 0 &&
                    env(kEnvAttnOSeparate) == nullptr;
  if (!fuse) {
    float* att = (float*)b;
    const size_t a = align256((size_t)count * (size_t)H * 4);
    QMM_TRY(qmm_prefill_attention(q, ldq, kcache, vcache, first, count, att, H, heads, kv_heads, head_dim, max_seq,
                                  scale, stream));
    const qmm_qtensor* w1[1] = {wo};
    float* y1[1] = {x};
    const int64_t l1[1] = {ldx};
    return qmm_matmul_ex(w1, 1, att, count, H, nullptr, 0.0f, 1, y1, l1, b + a, ws_bytes - a, stream);
  }
  const Planes pl = mmq_planes(wo->dtype, count, H);
  const int gt = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
  char name[64];
  snprintf(name, sizeof(name), "qmm_prefill_attention_planes_d%d_g%d", head_dim / 64, gt);
  long long a = ldq;
  int f = (int)first, kq = (int)H;
  void* q8 = b + pl.q8;
  void* dd = b + pl.d;
  void* ss = b + pl.s;
  void* args[] = {&q, &a, &kcache, &vcache, &f, &q8, &dd, &ss, &kq, &heads, &kv_heads, &max_seq, &scale};
  hipFunction_t fn;
  QMM_TRY(kernel(d, name, &fn));
  QMM_HIP(hipModuleLaunchKernel(fn, (unsigned)kv_heads, (unsigned)count, 1, 256, 1, 1, 0, s, args, nullptr));
  // the GEMM as matmul_targets runs it: planes first, split partials in the rest
  return gemm(d, wo, b, count, x, ldx, nullptr, s, 1, (float*)(b + pl.total), ws_bytes - pl.total);
}

int qmm_stream_read(const void* data, size_t bytes, uint32_t* sink, int variant, int wgs_per_cu, void* stream) {
  if (!data || !sink || bytes == 0 || bytes % 16) return fail(QMM_ERR_INVALID, "stream_read: bytes must be a positive multiple of 16");
  static const char* const names[] = {"qmm_stream_read_gs4", "qmm_stream_read_gs8", "qmm_stream_read_ch8nt"};
  if (variant < 0 || variant > 2) return fail(QMM_ERR_INVALID, "stream_read: variant must be 0 (gs4), 1 (gs8) or 2 (ch8nt)");
  if (wgs_per_cu < 0 || wgs_per_cu > 64) return fail(QMM_ERR_INVALID, "stream_read: wgs_per_cu must be in [0, 64]");
  Device* d;
  QMM_TRY(current_device(&d));
  long long n16 = (long long)(bytes / 16);
  const int per = wgs_per_cu > 0 ? wgs_per_cu : 8;
  void* args[] = {&data, &n16, &sink};
  return launch(d, names[variant], (unsigned)(d->num_cu * per), 256, 0, (hipStream_t)stream, args);
}

int qmm_silu_mul(const float* g, const float* u, float* h, int64_t n, void* stream) {
  if (!g || !u || !h || n < 0) return fail(QMM_ERR_INVALID, "bad silu_mul arguments");
  if (n == 0) return QMM_OK;
  Device* d;
  QMM_TRY(current_device(&d));
  long long nn = n;
  void* args[] = {&g, &u, &h, &nn};
  return launch(d, "qmm_silu_mul", ceil_div(n, 256), 256, 0, (hipStream_t)stream, args);
}

int qmm_silu_mul_quantize(const float* g, const float* u, int64_t rows, int64_t k, int64_t ld, void* hq,
                          void* stream) {
  if (!g || !u || !hq || rows < 1 || k < 256 || k % 256 || ld < k) return fail(QMM_ERR_INVALID, "bad silu_mul arguments");
  Device* d;
  QMM_TRY(current_device(&d));
  long long l = ld;
  int kk = (int)k, rr = (int)rows;
  void* args[] = {&g, &u, &l, &hq, &kk, &rr};
  return launch(d, "qmm_silu_mul_q8k", ceil_div(rows * (k / 256), 4), 256, 0, (hipStream_t)stream, args);
}

// Workgroups of the argmax (256 threads each). Each workgroup's slice result
// costs a device-scope fence (an L2 writeback) and an atomic: 512 workgroups,
// one logit per thread, measured 17 us against 10.6 us for 128.
static const int kArgmaxBlocks = 128;

size_t qmm_greedy_workspace_size(int64_t n) {
  (void)n;
  return 256 + (size_t)kArgmaxBlocks * 8;
}

int qmm_greedy_advance(const float* logits, int64_t n, int32_t* tokens, int64_t capacity, int32_t* pos,
                       int prompt_len, void* ws, size_t ws_bytes, void* stream) {
  if (!logits || !tokens || !pos || n < 1 || n > INT32_MAX || capacity < 1 || capacity > INT32_MAX)
    return fail(QMM_ERR_INVALID, "bad argmax arguments");
  const size_t need = qmm_greedy_workspace_size(n);
  if (!ws || ws_bytes < need) return fail(QMM_ERR_INVALID, "argmax workspace of %zu B < %zu B", ws_bytes, need);
  Device* d;
  QMM_TRY(current_device(&d));
  int nn = (int)n, cap = (int)capacity;
  unsigned* counter = (unsigned*)ws;
  float* pval = (float*)((uint8_t*)ws + 256);
  int* pidx = (int*)(pval + kArgmaxBlocks);
  void* args[] = {&logits, &nn, &tokens, &cap, &pos, &prompt_len, &pval, &pidx, &counter};
  return launch(d, "qmm_decode_argmax", kArgmaxBlocks, 256, 0, (hipStream_t)stream, args);
}

int qmm_block_dots(const qmm_qtensor* w, const void* xq, int64_t m, float* y, int64_t ldy, int32_t* dots, void* ws,
                   size_t ws_bytes, void* stream) {
  QMM_TRY(check_matmul(w, m, y, ldy));
  if (!xq || !dots) return fail(QMM_ERR_INVALID, "null pointer");
  Device* d;
  QMM_TRY(current_device(&d));
  if (m > 8) return gemm_from_blocks(d, w, xq, m, y, ldy, dots, ws, ws_bytes, (hipStream_t)stream);
  GemvTarget t = {w, y, ldy};
  return gemv(d, &t, 1, xq, false, 0, (int)m, dots, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// mixture of experts
// ---------------------------------------------------------------------------

static int route_check(int64_t tokens, int experts, int topk, float routed_scaling_factor) {
  if (tokens < 1 || tokens > 4096 || experts < 1 || experts > 256 || topk < 1 || topk > 8 || topk > experts ||
      tokens * topk > 8192)
    return fail(QMM_ERR_INVALID, "routing limits: 1 <= tokens <= 4096, tokens*topk <= 8192, topk <= min(8, experts)");
  if (!(routed_scaling_factor == routed_scaling_factor)) return fail(QMM_ERR_INVALID, "routed scaling factor is NaN");
  return QMM_OK;
}

int qmm_moe_route_ex(const float* logits, int64_t tokens, int experts, int topk, int renormalize,
                     float routed_scaling_factor, int32_t* counts, int32_t* offsets, int32_t* pair_token,
                     float* pair_weight, int32_t* token_pairs, void* stream) {
  if (!logits || !counts || !offsets || !pair_token || !pair_weight || !token_pairs)
    return fail(QMM_ERR_INVALID, "null pointer");
  QMM_TRY(route_check(tokens, experts, topk, routed_scaling_factor));
  Device* d;
  QMM_TRY(current_device(&d));
  int T = (int)tokens, E = experts, k = topk, rn = renormalize ? 1 : 0;
  float ps = routed_scaling_factor;
  void* args[] = {&logits, &T, &E, &k, &rn, &ps, &counts, &offsets, &pair_token, &pair_weight, &token_pairs};
  return launch(d, "qmm_moe_route", 1, 256, 0, (hipStream_t)stream, args);
}

int qmm_moe_route(const float* logits, int64_t tokens, int experts, int topk, int renormalize, int32_t* counts,
                  int32_t* offsets, int32_t* pair_token, float* pair_weight, int32_t* token_pairs, void* stream) {
  return qmm_moe_route_ex(logits, tokens, experts, topk, renormalize, 1.0f, counts, offsets, pair_token, pair_weight,
                          token_pairs, stream);
}

// max_count bounds every counts[e] (the token count under top-k routing, else
// the pair count): the ring kernel runs one 8-token pass per workgroup, grid y
// = the passes an expert can need.
// Token rows per pass of the matrix-core expert GEMV (qmm_moe_gemvm_q4k) for
// weights of w's K: up to 16, as many as the staged rows' LDS allows.
static int moe_gemvm_rows(const Device* d, const qmm_qtensor* w) {
  const long long K = w->k, nb = K / 256;
  return (int)std::min<long long>(16, (d->max_lds - 320LL * nb - 2048) / (K + 16));
}

// The matrix-core expert GEMV (Q4_K experts) over Q8_K rows at xq: passes of
// moe_gemvm_rows tokens up to a bound of max_count per expert.
static int moe_gemvm(Device* d, const qmm_qtensor* const* w, int count, int experts, const void* xq, int64_t pairs,
                     int64_t max_count, const int32_t* counts, const int32_t* offsets, float* const* y,
                     hipStream_t s) {
  int K = (int)w[0]->k;
  const int nb = K / 256, mt = moe_gemvm_rows(d, w[0]);
  const long long gpasses = (std::max<long long>(std::min<long long>(max_count, pairs), 1) + mt - 1) / mt;
  const int vt = qmm_vec_dot_type(w[0]->dtype);
  long long xrow = (w[0]->k / qmm_block_size(vt)) * qmm_type_size(vt);
  int N = (int)(w[0]->n / experts), E = experts, nj = count, ld = N, mtt = mt;
  const void* w0 = w[0]->data;
  const void* w1 = count > 1 ? w[1]->data : w[0]->data;
  float* y0 = y[0];
  float* y1 = count > 1 ? y[1] : y[0];
  const void* xp = xq;
  void* args[] = {&w0, &w1, &nj, &N, &E, &y0, &y1, &ld, &xp, &xrow, &counts, &offsets, &K, &mtt};
  hipFunction_t f;
  QMM_TRY(kernel(d, "qmm_moe_gemvm_q4k_w4_p4", &f));
  const long long gr = std::max<long long>((long long)d->num_cu * 4, E);
  QMM_HIP(hipModuleLaunchKernel(f, (unsigned)gr, (unsigned)gpasses, 1, 256, 1, 1,
                                (unsigned)(mt * (K + 16) + 320 * nb), s, args, nullptr));
  return QMM_OK;
}

static int moe_gemv(const qmm_qtensor* const* w, int count, int experts, const void* xq, int64_t pairs,
                    int64_t max_count, const int32_t* counts, const int32_t* offsets, float* const* y, void* stream) {
  if (!w || !y || !xq || !counts || !offsets || count < 1 || count > 2)
    return fail(QMM_ERR_INVALID, "need 1..2 stacked weights, activations, routing arrays and outputs");
  if (experts < 1 || experts > 65535) return fail(QMM_ERR_INVALID, "bad expert count %d", experts);
  for (int j = 0; j < count; ++j) {
    if (!w[j] || !y[j]) return fail(QMM_ERR_INVALID, "null weight or output");
    if (w[j]->dtype != w[0]->dtype || w[j]->k != w[0]->k || w[j]->n != w[0]->n)
      return fail(QMM_ERR_INVALID, "stacked expert weights must share dtype and shape");
  }
  if (w[0]->n % experts) return fail(QMM_ERR_INVALID, "rows %lld not divisible by %d experts", (long long)w[0]->n, experts);
  Device* d;
  QMM_TRY(current_device(&d));
  const int fmt = fmt_of(w[0]->dtype);
  const int nb = (int)(w[0]->k / qmm_block_size(w[0]->dtype));
  const int bpi = fmt == kFmtQ80 ? 64 : 16;
  const int niter = (nb + bpi - 1) / bpi;
  const unsigned lds = (unsigned)(8 * nb * (fmt == kFmtQ80 ? 36 : 292));
  if ((int)lds > d->max_lds) return fail(QMM_ERR_UNSUPPORTED, "expert activation needs %u B of LDS", lds);
  // k-quants: the one-row ring kernels (16 waves, two workgroups per CU when
  // every expert is active); QMM_MOE_GEMV=0 selects the generic M = 8 GEMV,
  // QMM_MOE_GEMV=<P> the ring depth.
  int ring = fmt == kFmtQ4K || fmt == kFmtQ6K ? 1 : 0;  // depth 2 measured no faster (Q4_K up to 3% slower)
  if (const char* e = env(kEnvMoeGemv)) ring = fmt != kFmtQ80 ? std::min(std::max(atoi(e), 0), 2) : 0;
  if (experts > 256) ring = 0;  // the ring kernel lists the active experts in a 256-entry LDS table
  // the ring kernel addresses an expert's rows with 32-bit offsets
  const unsigned long long body = fmt == kFmtQ4K ? 144 : 208;  // device block bodies (Q6_K's f16 d kept apart)
  if ((unsigned long long)(w[0]->n / experts) * (unsigned long long)nb * body >= (1ull << 32)) ring = 0;
  const long long passes = (std::max<long long>(std::min<long long>(max_count, pairs), 1) + 7) / 8;
  if (passes > 64) ring = 0;  // many idle pass workgroups: the generic kernel loops over its rows instead
  // Q4_K experts averaging six or more routed pairs: the matrix-core
  // multi-token GEMV (qmm_moe_gemvm_q4k, passes of up to 16 tokens; 305 vs
  // 377 us for a 32-token top-2 FFN over 8 Mixtral-shape experts, slower
  // than the ring kernel at two to four tokens per expert). QMM_GEMVM=0
  // never, 1 for every Q4_K call the ring kernel would take.
  int gvm = -1;
  if (const char* e = env(kEnvGemvm)) gvm = atoi(e);
  if (ring && fmt == kFmtQ4K && (gvm > 0 || (gvm < 0 && pairs >= 6LL * experts)) && moe_gemvm_rows(d, w[0]) >= 1)
    return moe_gemvm(d, w, count, experts, xq, pairs, max_count, counts, offsets, y, (hipStream_t)stream);
  char name[48];
  if (ring)
    snprintf(name, sizeof(name), "qmm_moe_gemv1_%s_p%d", fmt_name(fmt), ring);
  else
    snprintf(name, sizeof(name), "qmm_moe_gemv_%s_u%d", fmt_name(fmt), niter >= 2 ? 2 : 1);
  const int vt = qmm_vec_dot_type(w[0]->dtype);
  long long xrow = (w[0]->k / qmm_block_size(vt)) * qmm_type_size(vt);
  int N = (int)(w[0]->n / experts), E = experts, nj = count, K = (int)w[0]->k, ld = N;
  const void* w0 = w[0]->data;
  const void* w1 = count > 1 ? w[1]->data : w[0]->data;
  float* y0 = y[0];
  float* y1 = count > 1 ? y[1] : y[0];
  const void* xp = xq;
  void* args[] = {&w0, &w1, &nj, &N, &E, &y0, &y1, &ld, &xp, &xrow, &counts, &offsets, &K};
  // generic: ~20 resident waves per CU spread over the experts (grid y =
  // expert, idle experts exit at once); ring: per pass (grid y), 2 * CUs
  // 16-wave workgroups shared out over that pass's experts inside the kernel
  // (grid x >= E)
  const int wpg = ring ? 16 : 8;
  hipFunction_t f;
  QMM_TRY(kernel(d, name, &f));
  if (ring) {
    const long long gr = std::max<long long>((long long)d->num_cu * 2, E);
    QMM_HIP(hipModuleLaunchKernel(f, (unsigned)gr, (unsigned)passes, 1, 64 * wpg, 1, 1, lds, (hipStream_t)stream,
                                  args, nullptr));
    return QMM_OK;
  }
  long long gx = ((long long)d->num_cu * 20 / 8 + E - 1) / E;
  const long long need = ((long long)N * count + wpg - 1) / wpg;
  if (gx > need) gx = need;
  if (gx < 1) gx = 1;
  QMM_HIP(hipModuleLaunchKernel(f, (unsigned)gx, (unsigned)E, 1, 64 * wpg, 1, 1, lds, (hipStream_t)stream, args,
                                nullptr));
  return QMM_OK;
}

int qmm_moe_gemv(const qmm_qtensor* const* w, int count, int experts, const void* xq, int64_t pairs,
                 const int32_t* counts, const int32_t* offsets, float* const* y, void* stream) {
  return moe_gemv(w, count, experts, xq, pairs, pairs, counts, offsets, y, stream);
}

// Grouped prefill GEMM over expert-ordered f32 rows: the rows are quantized
// into GEMM planes in `ws`, then one launch per weight runs every expert's
// M tiles (grid z = expert; tiles past an expert's rows exit at once).
size_t qmm_moe_gemm_workspace_size(const qmm_qtensor* w, int64_t pairs) {
  if (!w || pairs < 1) return 0;
  return mmq_planes(w->dtype, pairs, w->k).total;
}

static int moe_gemm_planes(Device* d, const qmm_qtensor* const* w, int count, int experts, const uint8_t* planes,
                           int64_t pairs, int64_t max_rows, const int32_t* counts, const int32_t* offsets,
                           float* const* y, hipStream_t s, float* part = nullptr, size_t part_bytes = 0,
                           bool whole_tiles = false);

int qmm_moe_gemm(const qmm_qtensor* const* w, int count, int experts, const float* x, int64_t pairs, int64_t ldx,
                 int64_t max_rows, const int32_t* counts, const int32_t* offsets, float* const* y, void* ws,
                 size_t ws_bytes, void* stream) {
  if (!w || !y || !x || !counts || !offsets || !ws || count < 1 || count > 2)
    return fail(QMM_ERR_INVALID, "need 1..2 stacked weights, rows, routing arrays, outputs and a workspace");
  if (experts < 1 || experts > 65535) return fail(QMM_ERR_INVALID, "bad expert count %d", experts);
  for (int j = 0; j < count; ++j) {
    if (!w[j] || !y[j]) return fail(QMM_ERR_INVALID, "null weight or output");
    if (w[j]->dtype != w[0]->dtype || w[j]->k != w[0]->k || w[j]->n != w[0]->n)
      return fail(QMM_ERR_INVALID, "stacked expert weights must share dtype and shape");
  }
  const qmm_qtensor* w0 = w[0];
  if (w0->n % experts) return fail(QMM_ERR_INVALID, "rows %lld not divisible by %d experts", (long long)w0->n, experts);
  if (w0->k % 256) return fail(QMM_ERR_UNSUPPORTED, "grouped GEMM needs k %% 256 == 0 (k = %lld)", (long long)w0->k);
  if (pairs < 1 || pairs > (1LL << 24) || ldx < w0->k)
    return fail(QMM_ERR_INVALID, "pairs must be 1..2^24 and ldx >= k");
  if (max_rows < 1 || max_rows > pairs) return fail(QMM_ERR_INVALID, "max_rows must be 1..pairs");
  if (ws_bytes < qmm_moe_gemm_workspace_size(w0, pairs))
    return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, qmm_moe_gemm_workspace_size(w0, pairs));
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* b = (uint8_t*)ws;
  QMM_TRY(quantize_planes(d, w0->dtype, x, pairs, w0->k, ldx, b, s));
  return moe_gemm_planes(d, w, count, experts, b, pairs, max_rows, counts, offsets, y, s);
}

// The grouped GEMM launches over activation planes already at `planes`
// (mmq_planes(w[0]->dtype, pairs, k) layout). With `part` (part_bytes of
// scratch), the first-generation tile (Q6_K, Q8_0) splits K as the dense
// GEMM does, its split count from the same rounds x K-steps model over an
// estimate of the active tiles (each expert's rows padded to the 64-row
// tile: pairs / 64 + experts row tiles), and qmm_splitk_sum adds the
// partials in split order. The config-5 prefill's Q6_K down projection
// (1,024 pairs over 8 experts, ~640 active tiles on 512 resident slots)
// ran two rounds of 56 K steps, the second a quarter full; 2 splits run
// 2.5 rounds of 28. QMM_MOE_SPLITK=<S> forces S (0 or 1: unsplit).
static int moe_gemm_planes(Device* d, const qmm_qtensor* const* w, int count, int experts, const uint8_t* planes,
                           int64_t pairs, int64_t max_rows, const int32_t* counts, const int32_t* offsets,
                           float* const* y, hipStream_t s, float* part, size_t part_bytes, bool whole_tiles) {
  const qmm_qtensor* w0 = w[0];
  const Planes pl = mmq_planes(w0->dtype, pairs, w0->k);
  const int fmt = fmt_of(w0->dtype);
  const void* q8 = planes + pl.q8;
  const void* dd = planes + pl.d;
  const void* ss = planes + pl.s;
  int N = (int)(w0->n / experts), K = (int)w0->k, ld = N, E = experts;
  // Q4_K: the split-scale mmqs tile (128 x 128, eight waves) as in the dense
  // GEMM; QMM_MOE_MMQ=2 selects the older mmq2 tile, 128 rows (QMM_MOE_BM=64:
  // 64-row tiles, less padding when an expert's row count sits just above a
  // multiple of 128)
  const unsigned ldss = 2u * (128 * 272 + 128 * 144 + 128 * 4 + 128 * 48 + 128 * 48 + 128 * 80);
  const char* gen = env(kEnvMoeMmq);
  const bool use_s = fmt == kFmtQ4K && (gen == nullptr || atoi(gen) != 2) && (int)ldss <= d->max_lds;
  int bm = 64;
  if (fmt == kFmtQ4K) {
    bm = 128;
    if (const char* e = env(kEnvMoeBm); e && !use_s) bm = atoi(e) == 64 ? 64 : 128;
  }
  const int bn = 128;
  unsigned lds = fmt == kFmtQ4K ? (unsigned)(2 * (bm * 272 + 128 * 144 + bm * 4 + bm * 16)) : 0u;
  unsigned threads = fmt == kFmtQ4K ? (unsigned)(bm * 4) : 256u;
  // Q6_K keeps the first-generation 64-row tile here: the split-digit tile's
  // 128-row tiles pad an expert's 129..143 rows to 256 (192 with 64-row
  // tiles), and the 512-token config-5 prefill ran 1,086-1,146 us with it
  // against 1,003-1,044 us
  // whole_tiles (the tails' split left most experts a multiple of 128 GEMM
  // rows): Q6_K on the split-digit tile
  const bool use_s6 = whole_tiles && fmt == kFmtQ6K && (int)(2 * kS6StageBytes) <= d->max_lds;
  char name[40];
  if (use_s) {
    snprintf(name, sizeof(name), "qmm_moe_mmqs_q4k");
    lds = ldss;
    threads = 512;
  } else if (use_s6) {
    snprintf(name, sizeof(name), "qmm_moe_mmqs6_q6k");
    bm = 128;
    lds = 2 * kS6StageBytes;
    threads = 512;
  } else if (fmt == kFmtQ4K) {
    snprintf(name, sizeof(name), "qmm_moe_mmq2_q4k%s", bm == 64 ? "_m64" : "");
  } else {
    snprintf(name, sizeof(name), "qmm_moe_mmq_%s", fmt_name(fmt));
  }
  hipFunction_t f;
  QMM_TRY(kernel(d, name, &f));
  if (fmt != kFmtQ4K) {
    const int nbk = K / 256;
    int sp = 1;
    if (const char* e = env(kEnvMoeSplitK)) {
      sp = std::max(1, atoi(e));
    } else if (part) {
      const long long tiles = (pairs / bm + experts) * ((N + bn - 1) / bn);
      const long long slots = (long long)d->num_cu * std::max(1u, (unsigned)d->max_lds / (use_s6 ? lds : kMmqStaticLds));
      long long best = -1;
      for (int c = 1; c <= std::min(8, nbk); ++c) {
        const int kcc = (nbk + c - 1) / c;
        if (c > 1 && kcc < 2) break;
        const long long cost = (tiles * c + slots - 1) / slots * kcc;
        if (best < 0 || cost < best) {
          best = cost;
          sp = c;
        }
      }
    }
    int kc = (nbk + sp - 1) / sp;
    sp = (nbk + kc - 1) / kc;
    if (sp > 1 && (part == nullptr || (size_t)sp * (size_t)pairs * (size_t)N * 4 > part_bytes)) {
      sp = 1;
      kc = nbk;
    }
    long long ysplit = sp > 1 ? pairs * N : 0;
    for (int j = 0; j < count; ++j) {
      const void* wq = w[j]->data;
      float* yy = sp > 1 ? part : y[j];
      void* args[] = {&wq, &q8, &dd, &ss, &yy, &N, &K, &ld, &E, &counts, &offsets, &kc, &ysplit};
      QMM_HIP(hipModuleLaunchKernel(f, (unsigned)((N + bn - 1) / bn), (unsigned)((max_rows + bm - 1) / bm),
                                    (unsigned)(experts * sp), threads, 1, 1, lds, s, args, nullptr));
      if (sp > 1) {
        const float* pp = part;
        int spl = sp, M = (int)pairs, acc = 0;
        float* yo = y[j];
        void* a2[] = {&pp, &spl, &M, &N, &yo, &ld, &acc};
        QMM_TRY(launch(d, "qmm_splitk_sum", ceil_div(pairs * N, 256), 256, 0, s, a2));
      }
    }
    return QMM_OK;
  }
  if (use_s && count == 2 && 2 * experts <= 65535) {
    // gate and up in one grid (grid z = 2 E): a partial last round of tiles once
    // instead of twice (config-5 prefill: 896 tiles per weight on 256 CUs)
    const void* w0 = w[0]->data;
    const void* w1 = w[1]->data;
    float* y0 = y[0];
    float* y1 = y[1];
    void* args[] = {&w0, &w1, &q8, &dd, &ss, &y0, &y1, &N, &K, &ld, &E, &counts, &offsets};
    hipFunction_t f2;
    QMM_TRY(kernel(d, "qmm_moe_mmqs2_q4k", &f2));
    QMM_HIP(hipModuleLaunchKernel(f2, (unsigned)((N + bn - 1) / bn), (unsigned)((max_rows + bm - 1) / bm),
                                  (unsigned)(2 * experts), threads, 1, 1, lds, s, args, nullptr));
    return QMM_OK;
  }
  for (int j = 0; j < count; ++j) {
    const void* wq = w[j]->data;
    float* yy = y[j];
    void* args[] = {&wq, &q8, &dd, &ss, &yy, &N, &K, &ld, &E, &counts, &offsets};
    QMM_HIP(hipModuleLaunchKernel(f, (unsigned)((N + bn - 1) / bn), (unsigned)((max_rows + bm - 1) / bm),
                                  (unsigned)experts, threads, 1, 1, lds, s, args, nullptr));
  }
  return QMM_OK;
}

// Grouped prefill tails (see qmm_moe_split_tails): at most this many rows per
// expert go to the expert GEMV; QMM_MOE_TAILS=0 keeps every row in the GEMM.
constexpr int kMoeTailRows = 16;
static bool moe_tails_enabled() {
  const char* e = env(kEnvMoeTails);
  return !(e && atoi(e) == 0);
}

// qmm_moe_ffn runs the grouped GEMMs (prefill) instead of the expert GEMVs
// when the routed pairs average more than this many rows per expert: the
// GEMV streams an expert's weights once per eight rows, the GEMM once per
// 128-row tile. QMM_MOE_GROUPED=0/1 forces the choice.
static bool moe_grouped(int64_t pairs, int experts) {
  if (const char* e = env(kEnvMoeGrouped)) return atoi(e) != 0;
  return pairs > 16LL * experts;
}

// Workspace of qmm_moe_ffn, carved in this order.
struct MoeWs {
  size_t counts, offsets, pair_token, pair_weight, token_pairs, xg, xq, g, u, h, hq, yp, planes;
  size_t tails;  // grouped prefill: per expert the GEMM rows, the tail rows and the tails' first row
  size_t shared, sg, shared_ws, shared_ws_bytes;  // the shared expert (qmm_moe_ffn_ex)
  size_t total;
};
// The optional shared expert of qmm_moe_ffn_ex: a dense gated MLP over every
// token, and its sigmoid gate vector.
struct MoeShared {
  const qmm_qtensor *gate = nullptr, *up = nullptr, *down = nullptr;
  const float* gate_w = nullptr;  // f32 [hidden] or null (ungated)
};
static MoeWs moe_ws(const qmm_qtensor* gate, const qmm_qtensor* down, int64_t T, int E, int k,
                    const MoeShared* sh = nullptr) {
  MoeWs w = {};
  const int64_t P = T * k, H = gate->k, F = gate->n / E;
  const int vg = qmm_vec_dot_type(gate->dtype), vd = qmm_vec_dot_type(down->dtype);
  size_t o = 0;
  auto take = [&o](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  w.counts = take(4 * E);
  w.offsets = take(4 * (E + 1));
  w.pair_token = take(4 * P);
  w.pair_weight = take(4 * P);
  w.token_pairs = take(4 * P);
  w.xg = take(4 * P * H);  // f32 gathered rows (Q8_0 experts, grouped GEMMs)
  w.xq = take(P * (H / qmm_block_size(vg)) * qmm_type_size(vg));
  w.g = take(4 * P * F);
  w.u = take(4 * P * F);
  w.h = take(4 * P * F);
  w.hq = take(P * (F / qmm_block_size(vd)) * qmm_type_size(vd));
  w.yp = take(4 * P * H);
  w.planes = take(std::max(mmq_planes(gate->dtype, P, H).total, mmq_planes(down->dtype, P, F).total));
  w.tails = take(4 * (3 * (size_t)E + 1));
  if (sh != nullptr && sh->gate != nullptr) {
    w.shared = take(4 * T * H);
    w.sg = take(4 * T);
    w.shared_ws_bytes = qmm_ffn_workspace_size(sh->gate, sh->up, sh->down, T, 0);
    w.shared_ws = take(w.shared_ws_bytes);
  }
  w.total = o;
  return w;
}

static int check_moe(const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, int E, int k) {
  if (!gate || !up || !down) return fail(QMM_ERR_INVALID, "null expert weight");
  if (E < 1 || k < 1 || k > 8 || k > E) return fail(QMM_ERR_INVALID, "bad experts/topk %d/%d", E, k);
  if (gate->dtype != up->dtype || gate->n != up->n || gate->k != up->k)
    return fail(QMM_ERR_INVALID, "gate and up must share dtype and shape");
  if (gate->n % E || down->n % E) return fail(QMM_ERR_INVALID, "stacked rows not divisible by %d experts", E);
  if (down->n / E != gate->k || down->k != gate->n / E)
    return fail(QMM_ERR_INVALID, "down must be [E*hidden, ffn] for gate/up [E*ffn, hidden]");
  return QMM_OK;
}

static int check_moe_shared(const qmm_qtensor* gate, const MoeShared& sh) {
  if (sh.gate == nullptr && sh.up == nullptr && sh.down == nullptr) {
    if (sh.gate_w != nullptr) return fail(QMM_ERR_INVALID, "a shared-expert gate vector without a shared expert");
    return QMM_OK;
  }
  if (!sh.gate || !sh.up || !sh.down) return fail(QMM_ERR_INVALID, "the shared expert needs gate, up and down");
  if (sh.gate->k != gate->k) return fail(QMM_ERR_INVALID, "shared expert input width differs from the experts'");
  if (sh.down->n != gate->k) return fail(QMM_ERR_INVALID, "shared expert output width differs from the hidden size");
  if (qmm_ffn_workspace_size(sh.gate, sh.up, sh.down, 1, 0) == 0)
    return fail(QMM_ERR_INVALID, "shared expert weights do not form a gated MLP: %s", qmm_last_error());
  return QMM_OK;
}

// Tokens per routing launch (qmm_moe_route: tokens <= 4096, tokens * topk <=
// 8192). qmm_moe_ffn runs longer token lists as consecutive chunks of this
// many tokens: tokens are routed and combined independently, so the chunks'
// outputs are the whole list's.
static int64_t moe_chunk(int topk) { return std::min<int64_t>(4096, 8192 / std::max(topk, 1)); }

size_t qmm_moe_ffn_workspace_size(const qmm_qtensor* gate, const qmm_qtensor* down, int64_t tokens, int experts,
                                  int topk) {
  if (!gate || !down || tokens < 1 || experts < 1 || topk < 1) return 0;
  return moe_ws(gate, down, std::min(tokens, moe_chunk(topk)), experts, topk).total;
}

size_t qmm_moe_ffn_ex_workspace_size(const qmm_qtensor* gate, const qmm_qtensor* down, int64_t tokens, int experts,
                                     int topk, const qmm_qtensor* shared_gate, const qmm_qtensor* shared_up,
                                     const qmm_qtensor* shared_down) {
  if (!gate || !down || tokens < 1 || experts < 1 || topk < 1) return 0;
  MoeShared sh;
  sh.gate = shared_gate;
  sh.up = shared_up;
  sh.down = shared_down;
  if (check_moe_shared(gate, sh) != QMM_OK) return 0;
  return moe_ws(gate, down, std::min(tokens, moe_chunk(topk)), experts, topk, &sh).total;
}

// Decode-sized MoE: gathered Q8_K rows through the expert GEMVs.
static int moe_gemv_path(Device* d, const MoeWs& L, uint8_t* b, const float* x, int64_t ldx, const int32_t* ptok,
                         int64_t T, int64_t P, int64_t H, int64_t F, int experts, const int32_t* counts,
                         const int32_t* offsets,
                         const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, hipStream_t s,
                         bool gathered) {
  void* stream = s;
  const int vg = qmm_vec_dot_type(gate->dtype);
  if (!gathered) {
    const void* xp = x;
    long long lx = ldx;
    const int32_t* rows = ptok;
    int kk = (int)H, nr = (int)P;
    if (vg == QMM_Q8K) {
      void* yq = b + L.xq;
      void* args[] = {&xp, &lx, &rows, &yq, &kk, &nr};
      QMM_TRY(launch(d, "qmm_quantize_q8k_gather", ceil_div(P * (H / 256), 4), 256, 0, s, args));
    } else {
      void* xg = b + L.xg;
      void* args[] = {&xp, &lx, &rows, &xg, &kk, &nr};
      QMM_TRY(launch(d, "qmm_gather_rows", ceil_div(P * H, 256), 256, 0, s, args));
      QMM_TRY(qmm_quantize_rows(vg, (const float*)xg, P, H, H, b + L.xq, stream));
    }
  }
  float* g = (float*)(b + L.g);
  float* u = (float*)(b + L.u);
  float* h = (float*)(b + L.h);
  {
    const qmm_qtensor* gw[2] = {gate, up};
    float* gy[2] = {g, u};
    QMM_TRY(moe_gemv(gw, 2, experts, b + L.xq, P, T, counts, offsets, gy, stream));
  }
  const int vd = qmm_vec_dot_type(down->dtype);
  if (vd == QMM_Q8K) {
    // silu(g) * u quantized in registers (the same f32 values, one launch)
    QMM_TRY(qmm_silu_mul_quantize(g, u, P, F, F, b + L.hq, stream));
  } else {
    long long n = P * F;
    void* args[] = {&g, &u, &h, &n};
    QMM_TRY(launch(d, "qmm_silu_mul", ceil_div(n, 256), 256, 0, s, args));
    QMM_TRY(qmm_quantize_rows(vd, h, P, F, F, b + L.hq, stream));
  }
  float* yp = (float*)(b + L.yp);
  const qmm_qtensor* dw[1] = {down};
  float* dy[1] = {yp};
  return moe_gemv(dw, 1, experts, b + L.hq, P, T, counts, offsets, dy, stream);
}

static int moe_ffn(const float* x, int64_t tokens, int64_t ldx, const float* logits, int experts, int topk,
                   int renormalize, float routed_scaling_factor, const qmm_qtensor* gate, const qmm_qtensor* up,
                   const qmm_qtensor* down, const MoeShared& sh, float* out, int64_t ldo, void* ws, size_t ws_bytes,
                   void* stream) {
  QMM_TRY(check_moe(gate, up, down, experts, topk));
  QMM_TRY(check_moe_shared(gate, sh));
  if (!x || !logits || !out || !ws) return fail(QMM_ERR_INVALID, "null pointer");
  if (tokens < 1) return fail(QMM_ERR_INVALID, "tokens must be >= 1");
  if (ldx < gate->k || ldo < gate->k) return fail(QMM_ERR_INVALID, "row strides must be >= hidden size");
  const int64_t chunk = moe_chunk(topk);
  if (tokens > chunk) {  // consecutive chunks through the same workspace, in stream order
    for (int64_t t0 = 0; t0 < tokens; t0 += chunk)
      QMM_TRY(moe_ffn(x + t0 * ldx, std::min(chunk, tokens - t0), ldx, logits + t0 * experts, experts, topk,
                      renormalize, routed_scaling_factor, gate, up, down, sh, out + t0 * ldo, ldo, ws, ws_bytes,
                      stream));
    return QMM_OK;
  }
  const int64_t H = gate->k, F = gate->n / experts, P = tokens * topk;
  const MoeWs L = moe_ws(gate, down, tokens, experts, topk, &sh);
  if (ws_bytes < L.total) return fail(QMM_ERR_INVALID, "workspace of %zu B < %zu B needed", ws_bytes, L.total);
  Device* d;
  QMM_TRY(current_device(&d));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* b = (uint8_t*)ws;
  int32_t* counts = (int32_t*)(b + L.counts);
  int32_t* offsets = (int32_t*)(b + L.offsets);
  int32_t* ptok = (int32_t*)(b + L.pair_token);
  float* pw = (float*)(b + L.pair_weight);
  int32_t* tpairs = (int32_t*)(b + L.token_pairs);
  const bool grouped = moe_grouped(P, experts) && H % 256 == 0 && F % 256 == 0;
  // decode-sized calls with Q8_K activations: routing and the Q8_K gather of the routed rows in one launch
  // (every workgroup routes the tokens itself; the same lists as qmm_moe_route's)
  const bool fused_route = !grouped && qmm_vec_dot_type(gate->dtype) == QMM_Q8K && P <= 256;
  if (fused_route) {
    QMM_TRY(route_check(tokens, experts, topk, routed_scaling_factor));
    int T = (int)tokens, E = experts, k = topk, rn = renormalize ? 1 : 0, hh = (int)H;
    float ps = routed_scaling_factor;
    long long lx = ldx;
    void* xq = b + L.xq;
    void* args[] = {&logits, &T, &E, &k, &rn, &ps, &counts, &offsets, &ptok, &pw, &tpairs, &x, &lx, &xq, &hh};
    QMM_TRY(launch(d, "qmm_moe_route_gather_q8k", ceil_div(P * (H / 256), 4), 256, 0, s, args));
  } else {
    QMM_TRY(qmm_moe_route_ex(logits, tokens, experts, topk, renormalize, routed_scaling_factor, counts, offsets, ptok,
                             pw, tpairs, stream));
  }
  float* g = (float*)(b + L.g);
  float* u = (float*)(b + L.u);
  float* h = (float*)(b + L.h);
  float* yp = (float*)(b + L.yp);
  if (grouped) {
    // prefill: gathered rows -> grouped GEMMs (an expert holds at most
    // `tokens` pairs: a token's top-k experts are distinct)
    const int vg = qmm_vec_dot_type(gate->dtype), vd = qmm_vec_dot_type(down->dtype);
    if (vg == QMM_Q8K && vd == QMM_Q8K) {
      // Q8_K activations: the gather and SiLU*mul write the GEMM planes
      // directly (the same values as quantizing the f32 rows)
      uint8_t* pw8 = b + L.planes;
      // Q4_K gate / up: an expert's rows past its last full 128-row GEMM tile,
      // when at most 16, go to the matrix-core expert GEMV instead of a
      // nearly empty tile (the split is made on the device from the counts)
      const bool tails = fmt_of(gate->dtype) == kFmtQ4K && moe_gemvm_rows(d, gate) >= kMoeTailRows &&
                         moe_tails_enabled();
      int32_t* cg = (int32_t*)(b + L.tails);
      int32_t* ct = cg + experts;
      int32_t* ot = ct + experts;
      if (tails) {
        int E = experts, tile = 128, mx = kMoeTailRows;
        void* a1[] = {&counts, &offsets, &E, &tile, &mx, &cg, &ct, &ot};
        QMM_TRY(launch(d, "qmm_moe_split_tails", ceil_div(experts, 256), 256, 0, s, a1));
        // Q8_K rows of every routed pair, the tails' activations
        const void* xp = x;
        long long lx = ldx;
        const int32_t* rows = ptok;
        void* yq = b + L.xq;
        int kk = (int)H, nr = (int)P;
        void* a2[] = {&xp, &lx, &rows, &yq, &kk, &nr};
        QMM_TRY(launch(d, "qmm_quantize_q8k_gather", ceil_div(P * (H / 256), 4), 256, 0, s, a2));
      }
      {
        const Planes pl = mmq_planes(gate->dtype, P, H);
        const void* xp = x;
        long long lx = ldx;
        const int32_t* rows = ptok;
        void* q8 = pw8 + pl.q8;
        void* dd = pw8 + pl.d;
        void* ss = pw8 + pl.s;
        int kk = (int)H, mm = (int)P;
        void* args[] = {&xp, &lx, &rows, &q8, &dd, &ss, &kk, &mm};
        QMM_TRY(launch(d, "qmm_quantize_q8k_mmq_rows", ceil_div(P * (H / 256), 4), 256, 0, s, args));
      }
      const qmm_qtensor* gw[2] = {gate, up};
      float* gy[2] = {g, u};
      QMM_TRY(moe_gemm_planes(d, gw, 2, experts, pw8, P, tokens, tails ? cg : counts, offsets, gy, s));
      if (tails) QMM_TRY(moe_gemvm(d, gw, 2, experts, b + L.xq, P, kMoeTailRows, ct, ot, gy, s));
      {
        const Planes pl = mmq_planes(down->dtype, P, F);
        long long ld = F;
        void* q8 = pw8 + pl.q8;
        void* dd = pw8 + pl.d;
        void* ss = pw8 + pl.s;
        int kk = (int)F, mm = (int)P;
        void* args[] = {&g, &u, &ld, &q8, &dd, &ss, &kk, &mm};
        QMM_TRY(launch(d, "qmm_silu_mul_q8k_mmq", ceil_div(P * (F / 256), 4), 256, 0, s, args));
      }
      // the f32 SiLU rows (L.h) are not used on this path: their P x F floats
      // hold the down GEMM's split partials (up to F / H splits)
      const qmm_qtensor* dw[1] = {down};
      float* dy[1] = {yp};
      QMM_TRY(moe_gemm_planes(d, dw, 1, experts, pw8, P, tokens, tails ? cg : counts, offsets, dy, s,
                              (float*)(b + L.h), (size_t)(4 * P * F), tails));
      if (tails) {
        // the tails' down projection: their SiLU*mul rows as Q8_K rows, then the expert GEMV
        long long ld = F;
        void* hq = b + L.hq;
        int kk = (int)F, E = experts, mx = kMoeTailRows;
        void* a3[] = {&g, &u, &ld, &hq, &kk, &E, &mx, &ct, &ot};
        QMM_TRY(launch(d, "qmm_silu_mul_q8k_ranges", ceil_div((long long)experts * kMoeTailRows * (F / 256), 4), 256,
                       0, s, a3));
        QMM_TRY(moe_gemv(dw, 1, experts, b + L.hq, P, kMoeTailRows, ct, ot, dy, stream));
      }
    } else {
      float* xg = (float*)(b + L.xg);
      {
        const void* xp = x;
        long long lx = ldx;
        const int32_t* rows = ptok;
        int kk = (int)H, nr = (int)P;
        void* args[] = {&xp, &lx, &rows, &xg, &kk, &nr};
        QMM_TRY(launch(d, "qmm_gather_rows", ceil_div(P * H, 256), 256, 0, s, args));
      }
      const qmm_qtensor* gw[2] = {gate, up};
      float* gy[2] = {g, u};
      QMM_TRY(qmm_moe_gemm(gw, 2, experts, xg, P, H, tokens, counts, offsets, gy, b + L.planes,
                           L.total - L.planes, stream));
      {
        long long n = P * F;
        void* args[] = {&g, &u, &h, &n};
        QMM_TRY(launch(d, "qmm_silu_mul", ceil_div(n, 256), 256, 0, s, args));
      }
      const qmm_qtensor* dw[1] = {down};
      float* dy[1] = {yp};
      QMM_TRY(qmm_moe_gemm(dw, 1, experts, h, P, F, tokens, counts, offsets, dy, b + L.planes,
                           L.total - L.planes, stream));
    }
  } else {
    QMM_TRY(moe_gemv_path(d, L, b, x, ldx, ptok, tokens, P, H, F, experts, counts, offsets, gate, up, down, s,
                          fused_route));
  }
  // the always-on shared expert over every token (LlamaMlp::forward) and its
  // sigmoid gate, added by the combine after the routed sum
  float* shared = nullptr;
  float* sg = nullptr;
  if (sh.gate != nullptr) {
    shared = (float*)(b + L.shared);
    QMM_TRY(qmm_ffn(sh.gate, sh.up, sh.down, x, tokens, ldx, nullptr, 0.0f, 0, shared, H, b + L.shared_ws,
                    L.shared_ws_bytes, stream));
    if (sh.gate_w != nullptr) {
      sg = (float*)(b + L.sg);
      const float* gw = sh.gate_w;
      long long lx = ldx;
      int hh = (int)H, tt = (int)tokens;
      void* args[] = {&x, &lx, &gw, &hh, &tt, &sg};
      QMM_TRY(launch(d, "qmm_moe_shared_gate", ceil_div(tokens, 4), 256, 0, s, args));
    }
  }
  {
    int T = (int)tokens, k = topk, N = (int)H, lo = (int)ldo;
    void* args[] = {&yp, &pw, &tpairs, &T, &k, &N, &out, &lo, &shared, &sg};
    QMM_TRY(launch(d, "qmm_moe_combine", ceil_div(tokens * H, 256), 256, 0, s, args));
  }
  return QMM_OK;
}

int qmm_moe_ffn(const float* x, int64_t tokens, int64_t ldx, const float* logits, int experts, int topk,
                const qmm_qtensor* gate, const qmm_qtensor* up, const qmm_qtensor* down, float* out, int64_t ldo,
                void* ws, size_t ws_bytes, void* stream) {
  return moe_ffn(x, tokens, ldx, logits, experts, topk, 1, 1.0f, gate, up, down, MoeShared(), out, ldo, ws, ws_bytes,
                 stream);
}

int qmm_moe_ffn_ex(const float* x, int64_t tokens, int64_t ldx, const float* logits, int experts, int topk,
                   int norm_topk_prob, float routed_scaling_factor, const qmm_qtensor* gate, const qmm_qtensor* up,
                   const qmm_qtensor* down, const qmm_qtensor* shared_gate, const qmm_qtensor* shared_up,
                   const qmm_qtensor* shared_down, const float* shared_gate_weight, float* out, int64_t ldo, void* ws,
                   size_t ws_bytes, void* stream) {
  MoeShared sh;
  sh.gate = shared_gate;
  sh.up = shared_up;
  sh.down = shared_down;
  sh.gate_w = shared_gate_weight;
  return moe_ffn(x, tokens, ldx, logits, experts, topk, norm_topk_prob, routed_scaling_factor, gate, up, down, sh, out,
                 ldo, ws, ws_bytes, stream);
}

}  // extern "C"
