// Allocation-free entry: the per-tensor fp8 pair with its amax partials in a
// device array of this library instead of a caller- or library-allocated
// buffer, for callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope device array: each GPU that runs this library holds
// its own copy (16 KB) until the process ends.  On the host its name is only a
// stand-in for the symbol; the device address comes from hipGetSymbolAddress,
// resolved once per device (with that device current) on the first call that
// targets it, and only that address is passed to kernels.  The amax kernel
// writes every partial the apply kernel reads (one per workgroup, nb of them),
// so nothing needs clearing between calls.  All calls on one GPU share the
// array: calls that overlap on one GPU (concurrent streams, or host threads
// launching at once) race on it and must be serialised by the caller.
#include <mutex>

#include "k3h_internal.h"

namespace {
constexpr int kMaxPartials = K3H_NOALLOC_MAX_NB;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kMaxPartials];

namespace {
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` runs on (the current
// device for the null stream).
int scratch_on(void* stream, float** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev)
                        : hipGetDevice(&dev);
  if (e != hipSuccess) return k3h_hip(e);
  if (dev < 0 || dev >= kMaxDevices) return K3H_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return k3h_hip(e);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return k3h_hip(e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return k3h_hip(e);
    if (back != hipSuccess) return k3h_hip(back);
    if (!p) return K3H_EINVAL;
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return K3H_OK;
}
}  // namespace

extern "C" {

K3H_API int k3h_quant_fp8_tensor_noalloc(k3h_ctx_t ctx, void* stream, int v2, const void* x,
                                         void* y, float* scale_out, int n, int nb) {
  if (!ctx || n < 0 || nb < 1 || nb > kMaxPartials) return K3H_EINVAL;
  if (!k3h_okp(x, 16) || !k3h_okp(y, 8) || (scale_out && !k3h_aligned(scale_out, 4)))
    return K3H_EINVAL;
  float* partials = nullptr;
  const int r = scratch_on(stream, &partials);
  if (r != K3H_OK) return r;
  return k3h_quant_fp8_tensor(ctx, stream, v2, x, y, scale_out, partials, n, nb);
}

}  // extern "C"
