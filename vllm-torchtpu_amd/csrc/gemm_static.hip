// qmoe_gemm_static: the grouped GEMM with its split-K workspace in a static
// device array (no allocation on any call).

#include <mutex>

#include "gemm_route.h"

// qmoe_gemm_static runs qmoe_gemm with its split-K workspace in `scratch`, a
// file-scope device array (each GPU the library runs on holds its own copy
// until the process ends), for callers that cannot allocate (code under
// graph capture, serving loops, harnesses that forbid hipMalloc). In host
// code `scratch` names a host-side stand-in, not the device copy: its
// address on a device comes from hipGetSymbolAddress, looked up once per
// device on that device's first call and kept in g_scratch. The partial sums
// are written before they are read on every call, so the array needs no
// clearing; calls that overlap on one GPU (two streams, two threads) share
// the array and race.

namespace {

constexpr int64_t kStaticScratchBytes = 64ll << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure).
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int64_t qmoe_gemm_static_scratch_bytes(void) { return kStaticScratchBytes; }

extern "C" int qmoe_gemm_static(const qmoe_gemm_desc* d, hipStream_t stream) {
  GemmParams p;
  const int st = qmoe_to_params(d, &p);
  if (st != QMOE_OK) return st;
  if (d->M == 0) return QMOE_OK;
  QmoeRoute r;
  const int rc = qmoe_route_of(d, p, &r);
  if (rc != QMOE_OK) return rc;
  if (r.ws_bytes > kStaticScratchBytes) return QMOE_ERR_SCRATCH;
  void* ws = nullptr;
  if (r.ws_bytes > 0) {
    ws = scratch_on_current_device();
    if (!ws) return QMOE_ERR_LAUNCH;
  }
  return qmoe_run_route(d, r, p, ws, r.ws_bytes, stream);
}
