// Typed wrappers: per-tensor fp8 pair (manifest op quant_fp8_tensor,
// k3-tp4-prefill-16k.json:407194: amax then apply, both grid (2048), block 256).
#include "k3h_internal.h"

namespace {
const char* quant_key(int v2) { return v2 ? "k3_quant_fp8_pair_v2" : "k3_quant_fp8_pair"; }
bool quant_args_ok(const void* x, int n, const void* partials, int nb) {
  return n >= 0 && nb >= 1 && nb <= 65535 && k3h_okp(x, 16) && k3h_okp(partials, 4);
}
}  // namespace

extern "C" {

K3H_API int k3h_quant_fp8_amax(k3h_ctx_t ctx, void* stream, int v2, const void* x, int n,
                               float* partials, int nb) {
  if (!ctx || !quant_args_ok(x, n, partials, nb)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(x).i32(n).ptr(partials);
  return k3h_run(ctx, quant_key(v2), v2 ? "kern_quant_fp8_amax_v2" : "kern_quant_fp8_amax",
                 (uint32_t)nb, 1, 1, 256, stream, a);
}

K3H_API int k3h_quant_fp8_apply(k3h_ctx_t ctx, void* stream, int v2, const void* x, void* y,
                                int n, const float* partials, int nb, float* scale_out) {
  if (!ctx || !quant_args_ok(x, n, partials, nb) || !k3h_okp(y, 8)) return K3H_EINVAL;
  if (scale_out && !k3h_aligned(scale_out, 4)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(x).ptr(y).i32(n).ptr(partials).i32(nb).ptr(scale_out);
  return k3h_run(ctx, quant_key(v2), v2 ? "kern_quant_fp8_apply_v2" : "kern_quant_fp8_apply",
                 (uint32_t)nb, 1, 1, 256, stream, a);
}

K3H_API int k3h_quant_fp8_tensor(k3h_ctx_t ctx, void* stream, int v2, const void* x, void* y,
                                 float* scale_out, float* partials, int n, int nb) {
  const int r = k3h_quant_fp8_amax(ctx, stream, v2, x, n, partials, nb);
  if (r != K3H_OK) return r;
  return k3h_quant_fp8_apply(ctx, stream, v2, x, y, n, partials, nb, scale_out);
}

}  // extern "C"
