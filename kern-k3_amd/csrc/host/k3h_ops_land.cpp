// Typed wrappers: landing kernels of the shared-expert MLP and the MoE latent
// RMSNorm.  The manifests launch land_situ_n33792 (k3-tp4-prefill-16k.json:
// 405746) and the l0-bf16 ops rms (399525), land_n3584 (400710),
// land_situ_n6144 (400768) and land_situ_n33792 (400660, k3_situ_bf16) on a
// grid (rows, ceil(n / 1024)) of 1024 threads, and land_situ_rms (406727) on
// 3 ceil(tokens / 16) blocks of 512.  The entries are correct under those grids;
// the typed calls here launch compact grids of 256-thread blocks sized to the
// work (the entries walk the flattened output), because on MI355X the manifest
// grids' idle waves cost more than the work itself.  Shapes off the vector
// paths keep the manifest grid.
#include "k3h_internal.h"

namespace {
constexpr uint32_t kBlock = 1024;
constexpr uint32_t kCompact = 256;
}  // namespace

extern "C" {

K3H_API int k3h_rms(k3h_ctx_t ctx, void* stream, const void* x, const void* gamma, void* o, int h,
                    int B) {
  if (!ctx || B < 0 || h <= 0) return K3H_EINVAL;
  const size_t al = (h % 8 == 0) ? 16 : 2;
  if (!k3h_okp(x, al) || !k3h_okp(gamma, al) || !k3h_okp(o, al)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(x).ptr(gamma).ptr(o).i32(h).i32(B);
  if (h % 8 == 0 && h <= 8192)  // one row per wave, 4 per workgroup
    return k3h_run(ctx, "k3_land", "kern_k3_rms", k3h_cdiv(B, kCompact / 64), 1, 1, kCompact,
                   stream, a);
  return k3h_run(ctx, "k3_land", "kern_k3_rms", (uint32_t)B, 1, 1, kBlock, stream, a);
}

K3H_API int k3h_land(k3h_ctx_t ctx, void* stream, const float* p, void* o, int n, int off, int ldc,
                     int B) {
  if (!ctx || B < 0 || n <= 0 || off < 0 || ldc < off + n) return K3H_EINVAL;
  const bool vec = ((n | off | ldc) & 3) == 0;
  if (!k3h_okp(p, vec ? 16 : 4) || !k3h_okp(o, vec ? 8 : 2)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(p).ptr(o).i32(n).i32(off).i32(ldc).i32(B);
  if (vec)  // 8 values per thread
    return k3h_run(ctx, "k3_land", "kern_k3_land", k3h_cdiv((int64_t)B * n, 8 * kCompact), 1, 1,
                   kCompact, stream, a);
  return k3h_run(ctx, "k3_land", "kern_k3_land", (uint32_t)B, k3h_cdiv(n, kBlock), 1, kBlock,
                 stream, a);
}

K3H_API int k3h_land_situ(k3h_ctx_t ctx, void* stream, int bf16_in, const void* p, void* act,
                          int n, int B) {
  if (!ctx || B < 0 || n <= 0 || bf16_in < 0 || bf16_in > 2) return K3H_EINVAL;
  const bool vec = (n & 7) == 0;
  if (!k3h_okp(p, vec ? 16 : (bf16_in ? 2 : 4)) || !k3h_okp(act, vec ? 16 : 2)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(p).ptr(act).i32(n).i32(B);
  const char* mod = bf16_in == 0 ? "k3_land" : bf16_in == 1 ? "k3_land_bf16" : "k3_situ_bf16";
  const char* ent = bf16_in == 0   ? "kern_k3_land_situ"
                    : bf16_in == 1 ? "kern_k3_land_situ_bf16"
                                   : "kern_k3_situ_bf16";
  if (vec)  // 8 values per thread
    return k3h_run(ctx, mod, ent, k3h_cdiv((int64_t)B * n, 8 * kCompact), 1, 1, kCompact, stream,
                   a);
  return k3h_run(ctx, mod, ent, (uint32_t)B, k3h_cdiv(n, kBlock), 1, kBlock, stream, a);
}

K3H_API int k3h_situ_rms(k3h_ctx_t ctx, void* stream, const void* sp, void* act, const void* lat,
                         const void* gam, void* ln, int n, int B, int h, int L, int tokens) {
  if (!ctx || B < 0 || L < 0 || n <= 0 || h <= 0 || tokens < 0) return K3H_EINVAL;
  // the grid must cover both jobs: 4 rms rows and 4 situ rows per ceil(tokens/16)
  const int64_t groups = (tokens + 15) / 16;
  if (4 * groups < B || 4 * groups < L) return K3H_EINVAL;
  const size_t as = (n % 8 == 0) ? 16 : 2, al = (h % 8 == 0) ? 16 : 2;
  if (!k3h_okp(sp, as) || !k3h_okp(act, as) || !k3h_okp(lat, al) || !k3h_okp(gam, al) ||
      !k3h_okp(ln, al))
    return K3H_EINVAL;
  if (groups == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(sp).ptr(act).ptr(lat).ptr(gam).ptr(ln).i32(n).i32(B).i32(h).i32(L);
  return k3h_run(ctx, "k3_land_fused", "kern_k3_situ_rms_bf16", (uint32_t)(3 * groups), 1, 1, 512,
                 stream, a);
}

}  // extern "C"
