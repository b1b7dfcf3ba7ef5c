// Typed wrappers: K1 residual family, the fused residual + RMSNorm + MXFP8 op,
// and the MX quant.  Grid and block are the manifest's: one 128-thread
// workgroup per row (grid ceil(tokens/4) = B rows for the K1 ops,
// k3-tp4-prefill-16k.json:406888; l0-bf16 json:401191, 401295, 401328).
#include <string>

#include "k3h_internal.h"

int k3h_run(k3h_ctx_t ctx, const char* module_key, const char* entry, uint32_t gx, uint32_t gy,
            uint32_t gz, uint32_t block, void* stream, const K3hArgs& a, uint32_t shmem) {
  if (!a.ok()) return K3H_EINVAL;
  k3h_fn_t fn = nullptr;
  const int r = k3h_ctx_function(ctx, module_key, entry, &fn);
  if (r != K3H_OK) return r;
  const uint32_t grid[3] = {gx, gy, gz};
  const uint32_t blk[3] = {block, 1, 1};
  return k3h_launch(fn, grid, blk, shmem, stream, a.data(), a.size());
}

namespace {

constexpr int kNbMax = 8;
constexpr uint32_t kResThreads = 128;

// Module key for the K1 family: LAND_BF16 and the compiled eps.
bool residual_key(bool land_bf16, float eps, std::string* key) {
  *key = "k3_residual_v2";
  if (land_bf16) *key += "+LAND_BF16=1";
  if (eps == 1e-5f) return true;
  if (eps == 1e-6f) { *key += "+K3_EPS=1e-6f"; return true; }
  return false;
}

// Shared checks of the K1 row entries.
int check_rows(const void* gamma, const void* normed, const void* blocks, const float* sw, int nb,
               int B) {
  if (B < 0 || nb < 0 || nb > kNbMax) return K3H_EINVAL;
  if (!k3h_okp(gamma, 16) || !k3h_okp(normed, 16)) return K3H_EINVAL;
  if (nb > 0 && (!k3h_okp(blocks, 16) || !k3h_okp(sw, 16))) return K3H_EINVAL;
  return K3H_OK;
}

}  // namespace

extern "C" {

K3H_API int k3h_land_add_attnres_rms(k3h_ctx_t ctx, void* stream, int land_bf16,
                                     const void* partial, const void* prefix,
                                     const void* blocks, const float* sw, const void* gamma,
                                     void* prefix2, void* normed, int nb, int snapshot, int B,
                                     float eps) {
  std::string key;
  if (!ctx || !residual_key(land_bf16 != 0, eps, &key)) return K3H_EINVAL;
  int r = check_rows(gamma, normed, blocks, sw, nb, B);
  if (r != K3H_OK) return r;
  if (!k3h_okp(partial, 16) || !k3h_okp(prefix2, 16)) return K3H_EINVAL;
  if (!snapshot && !k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(partial).ptr(prefix).ptr(blocks).ptr(sw).ptr(gamma).ptr(prefix2).ptr(normed);
  a.i32(nb).i32(snapshot).i32(B);
  return k3h_run(ctx, key.c_str(), "kern_k3_land_add_attnres_rms", (uint32_t)B, 1, 1,
                 kResThreads, stream, a);
}

K3H_API int k3h_land_add_attnres_rms_nb(k3h_ctx_t ctx, void* stream, const void* partial,
                                        const void* prefix, const void* blocks, const float* sw,
                                        const void* gamma, void* prefix2, void* normed, int nb,
                                        int snapshot, int B) {
  if (!ctx || nb < 1 || nb > kNbMax) return K3H_EINVAL;
  int r = check_rows(gamma, normed, blocks, sw, nb, B);
  if (r != K3H_OK) return r;
  if (!k3h_okp(partial, 16) || !k3h_okp(prefix2, 16)) return K3H_EINVAL;
  if (!snapshot && !k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  // nb <= kSplitNbMax (every nb): the 256-thread vector-split entry (the
  // manifest entry's outputs, every candidate held on chip)
  const bool split = nb <= kSplitNbMax;
  const std::string entry = (split ? "k3h_land_add_attnres_rms_nb" : "kern_k3_land_add_attnres_rms_nb") +
                            std::to_string(nb) + (split ? "s" : "");
  K3hArgs a;
  a.ptr(partial).ptr(prefix).ptr(blocks).ptr(sw).ptr(gamma).ptr(prefix2).ptr(normed);
  a.i32(nb).i32(snapshot).i32(B);
  return k3h_run(ctx, "k3_residual_nb+LAND_BF16=1", entry.c_str(), (uint32_t)B, 1, 1,
                 split ? kSplitThreads : kResThreads, stream, a);
}

K3H_API int k3h_attnres_rms(k3h_ctx_t ctx, void* stream, const void* prefix, void* blocks,
                            const float* sw, const void* gamma, void* normed, int nb,
                            int snapshot, int B, float eps) {
  std::string key;
  if (!ctx || !residual_key(false, eps, &key)) return K3H_EINVAL;
  int r = check_rows(gamma, normed, blocks, sw, nb, B);
  if (r != K3H_OK) return r;
  if (!k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (snapshot && nb < kNbMax && !k3h_okp(blocks, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(prefix).ptr(blocks).ptr(sw).ptr(gamma).ptr(normed).i32(nb).i32(snapshot).i32(B);
  return k3h_run(ctx, key.c_str(), "kern_k3_attnres_rms", (uint32_t)B, 1, 1, kResThreads, stream,
                 a);
}

K3H_API int k3h_land_add2(k3h_ctx_t ctx, void* stream, const float* p1, const float* p2,
                          const void* prefix2, void* hidden, int two, int B) {
  if (!ctx || B < 0) return K3H_EINVAL;
  if (!k3h_okp(p1, 16) || !k3h_okp(prefix2, 16) || !k3h_okp(hidden, 16)) return K3H_EINVAL;
  if (two && !k3h_okp(p2, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(p1).ptr(p2).ptr(prefix2).ptr(hidden).i32(two).i32(B);
  return k3h_run(ctx, "k3_residual_v2", "kern_k3_land_add2", (uint32_t)B, 1, 1,
                 kResThreads, stream, a);
}

K3H_API int k3h_moe_quant(k3h_ctx_t ctx, void* stream, const void* x, void* q, void* sf,
                          int rows, int cols) {
  if (!ctx || rows < 0 || cols < 0) return K3H_EINVAL;
  const int64_t n = (int64_t)rows * cols;
  if (n % 32 != 0) return K3H_EINVAL;
  if (n == 0) return K3H_OK;
  if (!k3h_okp(x, 16) || !k3h_okp(q, 8) || !k3h_okp(sf, 1)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(x).ptr(q).ptr(sf).i32(rows).i32(cols);
  return k3h_run(ctx, "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16",
                 "kern_k3_moe_quant", k3h_cdiv(n / 32, 256), 1, 1, 256, stream, a);
}

K3H_API int k3h_residual_rms_mxfp8(k3h_ctx_t ctx, void* stream, const void* x,
                                   const void* residual, const void* gamma, void* residual_out,
                                   void* q, void* sf, void* normed, float eps, int B) {
  if (!ctx || B < 0 || !(eps > 0.0f)) return K3H_EINVAL;
  if (!k3h_okp(x, 16) || !k3h_okp(residual, 16) || !k3h_okp(gamma, 16) ||
      !k3h_okp(residual_out, 16) || !k3h_okp(q, 8) || !k3h_okp(sf, 4))
    return K3H_EINVAL;
  if (normed && !k3h_aligned(normed, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(x).ptr(residual).ptr(gamma).ptr(residual_out).ptr(q).ptr(sf).ptr(normed);
  a.f32(eps).i32(B);
  // two rows per 256-thread workgroup
  return k3h_run(ctx, "k3h_fused", "k3h_residual_rms_mxfp8", k3h_cdiv(B, 2), 1, 1,
                 2 * kResThreads, stream, a);
}

K3H_API int k3h_stream_copy(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                            int64_t n16) {
  if (!ctx || n16 < 0) return K3H_EINVAL;
  if (n16 == 0) return K3H_OK;
  if (!k3h_okp(src, 16) || !k3h_okp(dst, 16) || n16 > (int64_t)0xffffffff * 256) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(src).ptr(dst).i64(n16);
  return k3h_run(ctx, "k3h_fused", "k3h_stream_copy", k3h_cdiv(n16, 256), 1, 1, 256, stream, a);
}

}  // extern "C"
