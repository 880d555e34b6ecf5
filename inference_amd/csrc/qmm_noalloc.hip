// qmm_matmul_noalloc: qmm_matmul with the workspace taken from device memory
// that the library holds for the life of the process, so that the call
// itself allocates nothing (for callers that cannot call hipMalloc: code
// under stream capture, tight serving loops, harnesses that forbid it).
//
// The memory is a file-scope __device__ array of this translation unit
// (compiled by hipcc for gfx950 and linked into libqmm.so), one copy per GPU.
// Its device address is resolved once per device with hipGetSymbolAddress at
// set-up -- qmm_init(device), or the entry point's first call on a device --
// and kept per device; host code only ever passes that address on (the
// array's name in host code is a host-side stand-in, not a device address).
// The kernels are qmm_matmul's own and take the address as their workspace
// argument.
//
// Every call on one GPU shares that GPU's array and finds the previous call's
// contents in it: qmm_matmul's workspace holds the quantized activation (or
// GEMM planes) and split-K partials, each written in full before it is read,
// so nothing needs clearing. Calls that overlap on one GPU (two streams, two
// threads) race on the array; callers order them on one stream.
#include <hip/hip_runtime.h>

#include <mutex>

#include "qmm.h"

static_assert(QMM_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");

static __device__ __align__(256) unsigned char scratch[QMM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kScratchBytes = QMM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch` per device

}  // namespace

// Error reporting shared with qmm_host.cpp (sets qmm_last_error()).
__attribute__((visibility("hidden"))) int qmm_internal_fail(int code, const char* msg);

// Resolves the array's address on the current device (once per device).
extern "C" __attribute__((visibility("hidden"))) int qmm_internal_noalloc_setup(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qmm_internal_fail(QMM_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return qmm_internal_fail(QMM_ERR_INVALID, "device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return qmm_internal_fail(QMM_ERR_HIP, "hipGetSymbolAddress(scratch) failed on this device");
    }
    g_ptr[dev] = p;
  }
  if (out) *out = g_ptr[dev];
  return QMM_OK;
}

extern "C" int qmm_matmul_noalloc(const qmm_qtensor* w, const float* x, int64_t m, int64_t ldx, float* y,
                                  int64_t ldy, void* stream) {
  if (!w) return qmm_internal_fail(QMM_ERR_INVALID, "null weight");
  if (m <= 0) return qmm_internal_fail(QMM_ERR_INVALID, "m must be positive");
  const size_t need = qmm_matmul_workspace_size(w, m);
  if (need > kScratchBytes)
    return qmm_internal_fail(QMM_ERR_INVALID,
                             "qmm_matmul_noalloc: this call needs more workspace than the library's "
                             "per-device scratch (qmm_matmul_workspace_size > QMM_NOALLOC_SCRATCH_BYTES = 64 MiB); "
                             "use qmm_matmul with a caller workspace");
  void* ws = nullptr;
  const int rc = qmm_internal_noalloc_setup(&ws);
  if (rc != QMM_OK) return rc;
  return qmm_matmul(w, x, m, ldx, y, ldy, ws, kScratchBytes, stream);
}
