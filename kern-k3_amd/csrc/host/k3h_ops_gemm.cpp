// Typed wrappers: the MoE expert GEMMs on the MX-scaled matrix cores (module
// k3h_moe_gemm) and their load-time weight layouts.  They stand where the
// reference's manifest launches prebuilt batched GEMMs: ops moe_fc1
// (k3-tp4-prefill-16k.json:405185; params w13s, w13_sfs, latent_q_all,
// latent_sf_all, fc1_out, fc1_sf, route_map, alpha, beta, num_non_exiting,
// total_padded, cta_batch, cta_limit) and moe_fc2 (405419; w2s, w2_sfs, fc1_out,
// fc1_sf, fc2_out, num_non_exiting, total_padded, cta_batch, cta_limit), and the
// load-time shuffles kern_k3_moe_w_shuffle / kern_k3_moe_sf_shuffle.  The
// weight arguments are this build's tiled layouts (k3h_moe_w_tile /
// k3h_moe_sf_tile), not the reference GEMMs' shuffled ones.
#include <algorithm>
#include <atomic>

#include "k3h_internal.h"

namespace {
constexpr uint32_t kBlock = 256, kBlockWide = 512;
constexpr int kTileN = 256, kTileNWide = 512, kStepK = 128;

// The kernels keep the tile's A scales (K / 32 bytes per row) in LDS: entries
// without a suffix take K <= 3584, the "_w" entries K <= 7168.
constexpr int kMaxK = 7168, kMaxKNarrow = 3584;

bool gemm_shape_ok(int E, int N, int K, int max_tiles) {
  return E > 0 && N > 0 && K > 0 && max_tiles >= 0 && N % kTileN == 0 && K % kStepK == 0 &&
         K <= kMaxK;
}

K3hArgs gemm_args(const void* a, const void* a_sf, const int* a_rows, const void* wt,
                  const void* wsf, const int* num_tiles, const int* cta_batch, int E, int N, int K,
                  int max_tiles) {
  K3hArgs args;
  args.ptr(a).ptr(a_sf).ptr(a_rows).ptr(wt).ptr(wsf).ptr(num_tiles).ptr(cta_batch);
  args.i32(E).i32(N).i32(K).i32(max_tiles);
  return args;
}

// Grid rows of a GEMM launch.  The kernel hands the live (tile, column block)
// items out per XCD (workgroups are dispatched round-robin over the 8 XCDs by
// linear id), the XCDs forming an xt x xc grid over (tiles, column blocks) with
// xt * xc = 8; XCD x then needs ceil(tiles / xt) * ceil(nc / xc) workgroups of
// its own.  The grid is sized for the largest such need over every split, so it
// covers the kernel whichever split it was built with.
uint32_t gemm_grid_rows(int max_tiles, int nc) {
  int64_t need = 0;
  for (int xc = 1; xc <= 8; xc *= 2) {
    const int64_t xt = 8 / xc;
    need = std::max<int64_t>(need, 8 * k3h_cdiv(max_tiles, xt) * k3h_cdiv(nc, xc));
  }
  return (uint32_t)k3h_cdiv(need, nc);
}

// Compute units of the device `stream` runs on (the current device for the null
// stream), cached per device.
int stream_cus(void* stream, int* cus) {
  static std::atomic<int> cache[64];
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev)
                        : hipGetDevice(&dev);
  if (e != hipSuccess) return k3h_hip(e);
  if (dev < 0 || dev >= 64) return K3H_EINVAL;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return k3h_hip(e);
    if (n <= 0) return K3H_EINVAL;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  *cus = n;
  return K3H_OK;
}

bool gemm_ptrs_ok(const void* a, const void* a_sf, const int* a_rows, const void* wt,
                  const void* wsf, const int* num_tiles, const int* cta_batch) {
  return k3h_okp(a, 16) && k3h_okp(a_sf, 4) && (a_rows == nullptr || k3h_aligned(a_rows, 4)) &&
         k3h_okp(wt, 16) && k3h_okp(wsf, 8) && k3h_okp(num_tiles, 4) && k3h_okp(cta_batch, 4);
}
}  // namespace

extern "C" {

K3H_API int k3h_moe_w_tile(k3h_ctx_t ctx, void* stream, const void* src, void* dst, int experts,
                           int n, int k, int gated) {
  if (!ctx || experts < 0 || n <= 0 || k <= 0 || n % 32 || k % 64 || (gated && n % 64))
    return K3H_EINVAL;
  if (!k3h_okp(src, 16) || !k3h_okp(dst, 16)) return K3H_EINVAL;
  const int64_t total = (int64_t)experts * (n / 32) * (k / 64) * 64;
  if (total == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(src).ptr(dst).i32(experts).i32(n).i32(k).i32(gated ? 1 : 0);
  const uint32_t grid = std::min<int64_t>(k3h_cdiv(total, kBlock), 65536);
  return k3h_run(ctx, "k3h_moe_gemm", "kern_k3h_moe_w_tile", grid, 1, 1, kBlock, stream, a);
}

K3H_API int k3h_moe_sf_tile(k3h_ctx_t ctx, void* stream, const void* src, void* dst, int experts,
                            int n, int k, int gated) {
  if (!ctx || experts < 0 || n <= 0 || k <= 0 || n % 128 || k % 128) return K3H_EINVAL;
  if (!k3h_okp(src, 1) || !k3h_okp(dst, 8)) return K3H_EINVAL;
  const int64_t total = (int64_t)experts * (n / 128) * (k / 128) * 64 * 4;
  if (total == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(src).ptr(dst).i32(experts).i32(n).i32(k).i32(gated ? 1 : 0);
  const uint32_t grid = std::min<int64_t>(k3h_cdiv(total, kBlock), 65536);
  return k3h_run(ctx, "k3h_moe_gemm", "kern_k3h_moe_sf_tile", grid, 1, 1, kBlock, stream, a);
}

K3H_API int k3h_moe_gemm_mx(k3h_ctx_t ctx, void* stream, int epilogue, const void* a,
                            const void* a_sf, const int* a_rows, const void* wt, const void* wsf,
                            const int* num_tiles, const int* cta_batch, int max_tiles, int E,
                            int N, int K, void* out, void* out_sf, const float* alpha,
                            const float* beta) {
  if (!ctx || !gemm_shape_ok(E, N, K, max_tiles)) return K3H_EINVAL;
  // Activation row offsets are 32-bit in the kernels: read in place, every padded
  // row of every tile must sit below 4 GiB.
  if (a_rows == nullptr && (int64_t)max_tiles * 128 * K > (int64_t)UINT32_MAX) return K3H_EINVAL;
  if (!gemm_ptrs_ok(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch)) return K3H_EINVAL;
  K3hArgs args = gemm_args(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles);
  const bool wide = K > kMaxKNarrow;
  const char* entry = nullptr;
  switch (epilogue) {
    case K3H_GEMM_F32:
      if (!k3h_okp(out, 4)) return K3H_EINVAL;
      args.ptr(out);
      entry = wide ? "kern_k3h_moe_gemm_f32_w" : "kern_k3h_moe_gemm_f32";
      break;
    case K3H_GEMM_BF16:
      if (!k3h_okp(out, 16)) return K3H_EINVAL;
      args.ptr(out);
      entry = wide ? "kern_k3h_moe_gemm_bf16_w" : "kern_k3h_moe_gemm_bf16";
      break;
    case K3H_GEMM_F32_SITU_TILING:
      if (!k3h_okp(out, 16)) return K3H_EINVAL;
      args.ptr(out);
      entry = wide ? "kern_k3h_moe_gemm_situ_acc_w" : "kern_k3h_moe_gemm_situ_acc";
      break;
    case K3H_GEMM_SITU_MX:
      if (!k3h_okp(out, 16) || !k3h_okp(out_sf, 2) || !k3h_okp(alpha, 4) || !k3h_okp(beta, 4))
        return K3H_EINVAL;
      args.ptr(out).ptr(out_sf).ptr(alpha).ptr(beta);
      entry = wide ? "kern_k3h_moe_gemm_situ_mx_w" : "kern_k3h_moe_gemm_situ_mx";
      break;
    default:
      return K3H_EINVAL;
  }
  if (max_tiles == 0) return K3H_OK;
  // f32 / bf16 epilogues on 512-column items: persistent 8-wave workgroups
  // (kern_k3h_moe_gemm2_*, one per CU, grid a multiple of the 8 XCDs) where the
  // shape allows them; else, and for the SiTU-GLU + MXFP8 epilogue and its f32 tiling, 256-column
  // items on 4-wave workgroups (two per CU).
  if ((epilogue == K3H_GEMM_F32 || epilogue == K3H_GEMM_BF16) && N % kTileNWide == 0 && K >= 2 * kStepK &&
      K <= kMaxKNarrow && k3h_aligned(out, 16)) {
    int cus = 0;
    if (const int rc = stream_cus(stream, &cus)) return rc;
    const uint32_t grid = (uint32_t)std::max(8, cus / 8 * 8);
    return k3h_run(ctx, "k3h_moe_gemm",
                   epilogue == K3H_GEMM_F32 ? "kern_k3h_moe_gemm2_f32" : "kern_k3h_moe_gemm2_bf16",
                   grid, 1, 1, kBlockWide, stream, args);
  }
  const uint32_t rows = gemm_grid_rows(max_tiles, N / kTileN);
  if (rows > 65535u) return K3H_EINVAL;
  return k3h_run(ctx, "k3h_moe_gemm", entry, (uint32_t)(N / kTileN), rows, 1, kBlock, stream, args);
}

K3H_API int k3h_moe_fc1(k3h_ctx_t ctx, void* stream, const void* w13t, const void* w13_sft,
                        const void* a_q, const void* a_sf, void* fc1_out, void* fc1_sf,
                        const int* route_map, const float* alpha, const float* beta,
                        const int* num_non_exiting, const int* total_padded, const int* cta_batch,
                        const int* cta_limit, int max_tiles, int E, int K, int inter) {
  (void)total_padded;
  (void)cta_limit;
  if (inter <= 0) return K3H_EINVAL;
  return k3h_moe_gemm_mx(ctx, stream, K3H_GEMM_SITU_MX, a_q, a_sf, route_map, w13t, w13_sft,
                         num_non_exiting, cta_batch, max_tiles, E, 2 * inter, K, fc1_out, fc1_sf,
                         alpha, beta);
}

K3H_API int k3h_moe_fc2(k3h_ctx_t ctx, void* stream, const void* w2t, const void* w2_sft,
                        const void* fc1_out, const void* fc1_sf, void* fc2_out,
                        const int* num_non_exiting, const int* total_padded, const int* cta_batch,
                        const int* cta_limit, int max_tiles, int E, int inter, int cols) {
  (void)total_padded;
  (void)cta_limit;
  return k3h_moe_gemm_mx(ctx, stream, K3H_GEMM_BF16, fc1_out, fc1_sf, nullptr, w2t, w2_sft,
                         num_non_exiting, cta_batch, max_tiles, E, cols, inter, fc2_out, nullptr,
                         nullptr, nullptr);
}

}  // extern "C"
