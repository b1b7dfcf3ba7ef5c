// Typed wrappers: router top-k / argmax (module k3_router_argmax) and the EP
// routing, permute, finalize and weight-layout entries (k3_moe_prefill_v4).
// Grids follow the manifest ops (k3-tp4-prefill-16k.json): router_topk 404788
// (grid rows, block 256), moe_route_count 404991 (ceil(T/256), 256),
// moe_route_tables 405046 (1, 1024), moe_route_scatter 405120 (ceil(T/256),
// 512), moe_finalize 405686 (ceil(T/2), 128).  topk selects the code object:
// 16 is the manifest build, 8 the "+TOPK=8" build.
#include <algorithm>
#include <string>

#include "k3h_internal.h"

namespace {
constexpr int kExperts = 224;
constexpr int kMaxE = 64;
constexpr int kRouteMaxBlocks = 256;  // RF_MAX_BLOCKS of k3h_moe_route_fused
const char* kMoeV4 = "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16";

bool topk_key(const char* base, int topk, std::string* key) {
  *key = base;
  if (topk == 16) return true;
  if (topk == 8) { *key += "+TOPK=8"; return true; }
  return false;
}
}  // namespace

extern "C" {

K3H_API int k3h_router_topk(k3h_ctx_t ctx, void* stream, int topk, const float* S,
                            const float* bias, const void* rs, int* idx, float* wts, int B) {
  std::string key;
  if (!ctx || B < 0 || !topk_key("k3_router_argmax", topk, &key)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  if (!k3h_okp(S, 4) || !k3h_okp(bias, 4) || !k3h_okp(rs, 2) || !k3h_okp(idx, 4) ||
      !k3h_okp(wts, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(S).ptr(bias).ptr(rs).ptr(idx).ptr(wts).i32(B);
  // one row per half-wave (the manifest entry kern_k3_router_topk idles three waves of four
  // and gives the live one a row alone)
  return k3h_run(ctx, key.c_str(), "k3h_router_topk_pairs", k3h_cdiv(B, 8), 1, 1, 256, stream, a);
}

K3H_API int k3h_argmax_f32(k3h_ctx_t ctx, void* stream, const float* logits, float* pmax,
                           int* pidx, long long* out, int B, int n, int parts) {
  if (!ctx || B < 0 || n < 0 || parts < 1 || parts > 65535) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  if (!k3h_okp(logits, 4) || !k3h_okp(pmax, 4) || !k3h_okp(pidx, 4) || !k3h_okp(out, 8))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(logits).ptr(pmax).ptr(pidx).i32(n);
  int r = k3h_run(ctx, "k3_router_argmax", "kern_k3_argmax_f32_partial", (uint32_t)B,
                  (uint32_t)parts, 1, 1024, stream, a);
  if (r != K3H_OK) return r;
  K3hArgs b;
  b.ptr(pmax).ptr(pidx).ptr(out).i32(parts);
  return k3h_run(ctx, "k3_router_argmax", "kern_k3_argmax_f32_final", (uint32_t)B, 1, 1, 64,
                 stream, b);
}

K3H_API int k3h_moe_route_count(k3h_ctx_t ctx, void* stream, int topk, const int* ids, int T,
                                int rank, int E, int* blockcount) {
  std::string key;
  if (!ctx || T < 0 || E < 1 || E > kMaxE || rank < 0 || !topk_key(kMoeV4, topk, &key))
    return K3H_EINVAL;
  if (T == 0) return K3H_OK;
  if (!k3h_okp(ids, 4) || !k3h_okp(blockcount, 4)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(ids).i32(T).i32(rank).i32(E).ptr(blockcount);
  return k3h_run(ctx, key.c_str(), "kern_k3_moe_route_count", k3h_cdiv(T, 256), 1, 1, 256,
                 stream, a);
}

K3H_API int k3h_moe_route_tables(k3h_ctx_t ctx, void* stream, const int* blockcount, int blocks,
                                 int E, int tile, int* blockoff, int* cta_batch, int* cta_limit,
                                 int* num_non_exiting, int* total_padded, int* route_map) {
  if (!ctx || blocks < 0 || E < 1 || E > kMaxE || tile != 128) return K3H_EINVAL;
  if (!k3h_okp(blockcount, 4) || !k3h_okp(blockoff, 4) || !k3h_okp(cta_batch, 4) ||
      !k3h_okp(cta_limit, 4) || !k3h_okp(num_non_exiting, 4) || !k3h_okp(total_padded, 4) ||
      !k3h_okp(route_map, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(blockcount).i32(blocks).i32(E).i32(tile).ptr(blockoff).ptr(cta_batch).ptr(cta_limit);
  a.ptr(num_non_exiting).ptr(total_padded).ptr(route_map);
  return k3h_run(ctx, kMoeV4, "kern_k3_moe_route_tables", 1, 1, 1, 1024, stream, a);
}

K3H_API int k3h_moe_route_scatter(k3h_ctx_t ctx, void* stream, int topk, const int* ids,
                                  const int* blockoff, int T, int rank, int E, int* route_map,
                                  int* exp2perm) {
  std::string key;
  if (!ctx || T < 0 || E < 1 || E > kMaxE || rank < 0 || !topk_key(kMoeV4, topk, &key))
    return K3H_EINVAL;
  if (T == 0) return K3H_OK;
  if (!k3h_okp(ids, 4) || !k3h_okp(blockoff, 4) || !k3h_okp(route_map, 4) || !k3h_okp(exp2perm, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(ids).ptr(blockoff).i32(T).i32(rank).i32(E).ptr(route_map).ptr(exp2perm);
  return k3h_run(ctx, key.c_str(), "kern_k3_moe_route_scatter", k3h_cdiv(T, 256), 1, 1, 512,
                 stream, a);
}

K3H_API int k3h_moe_route(k3h_ctx_t ctx, void* stream, int topk, const int* ids, int T, int rank,
                          int E, int* blockcount, int* blockoff, int* cta_batch, int* cta_limit,
                          int* num_non_exiting, int* total_padded, int* route_map, int* exp2perm,
                          int* sync) {
  std::string key;
  if (!ctx || T < 0 || E < 1 || E > kMaxE || rank < 0 || !topk_key(kMoeV4, topk, &key))
    return K3H_EINVAL;
  const int blocks = (int)k3h_cdiv(T, 256);
  if (blocks > kRouteMaxBlocks) return K3H_EINVAL;
  if (!k3h_okp(blockcount, 4) || !k3h_okp(blockoff, 4) || !k3h_okp(cta_batch, 4) ||
      !k3h_okp(cta_limit, 4) || !k3h_okp(num_non_exiting, 4) || !k3h_okp(total_padded, 4) ||
      !k3h_okp(route_map, 4) || (T > 0 && !k3h_okp(ids, 4)) || (T > 0 && !k3h_okp(exp2perm, 4)) ||
      !k3h_okp(sync, 4))
    return K3H_EINVAL;
  if (T == 0)  // no ids: the tables of zero blocks (num_non_exiting = total_padded = 0)
    return k3h_moe_route_tables(ctx, stream, blockcount, 0, E, 128, blockoff, cta_batch, cta_limit,
                                num_non_exiting, total_padded, route_map);
  // the grid barrier needs every workgroup resident at once: refuse a device that
  // cannot hold the grid instead of relying on the kernel's bounded wait
  int resident = 0;
  const int rr = k3h_ctx_resident(ctx, key.c_str(), "k3h_moe_route_fused", 512, &resident);
  if (rr != K3H_OK) return rr;
  if (resident < blocks) return K3H_ERESIDENT;
  K3hArgs a;
  a.ptr(ids).i32(T).i32(rank).i32(E).ptr(blockcount).ptr(blockoff).ptr(cta_batch).ptr(cta_limit);
  a.ptr(num_non_exiting).ptr(total_padded).ptr(route_map).ptr(exp2perm).ptr(sync);
  return k3h_run(ctx, key.c_str(), "k3h_moe_route_fused", (uint32_t)blocks, 1, 1, 512, stream, a);
}

K3H_API int k3h_moe_finalize(k3h_ctx_t ctx, void* stream, int topk, const void* fc2,
                             const int* exp2perm, const float* wts, void* out, int T, int cols) {
  std::string key;
  if (!ctx || T < 0 || cols <= 0 || cols % 8 || !topk_key(kMoeV4, topk, &key)) return K3H_EINVAL;
  if (T == 0) return K3H_OK;
  if (!k3h_okp(fc2, 16) || !k3h_okp(exp2perm, 4) || !k3h_okp(wts, 4) || !k3h_okp(out, 16))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(fc2).ptr(exp2perm).ptr(wts).ptr(out).i32(T).i32(cols);
  // one 448-thread workgroup per token (k3h_moe_finalize_rows, the same bits as
  // the manifest entry kern_k3_moe_finalize, which gives each token one wave)
  return k3h_run(ctx, key.c_str(), "k3h_moe_finalize_rows", (uint32_t)T, 1, 1, 448, stream, a);
}

K3H_API int k3h_moe_permute_mx(k3h_ctx_t ctx, void* stream, const void* q, const void* sf,
                               const int* route_map, const int* total_padded, int max_rows,
                               int cols, void* pq, void* psf) {
  if (!ctx || cols <= 0 || cols % 1024 || cols > 16384 || max_rows < 0) return K3H_EINVAL;
  if (max_rows == 0) return K3H_OK;
  if (!k3h_okp(q, 16) || !k3h_okp(sf, 4) || !k3h_okp(route_map, 4) || !k3h_okp(total_padded, 4) ||
      !k3h_okp(pq, 16) || !k3h_okp(psf, 4))
    return K3H_EINVAL;
  K3hArgs a;
  a.ptr(q).ptr(sf).ptr(route_map).ptr(total_padded).i32(max_rows).i32(cols).ptr(pq).ptr(psf);
  // one row per wave; rows past *total_padded exit, and past 64K rows (max_rows is
  // often a capacity) the waves stride instead of launching empty workgroups
  const uint32_t grid = std::min<uint32_t>(k3h_cdiv(max_rows, 4), 16384u);
  return k3h_run(ctx, kMoeV4, "k3h_moe_permute_mx", grid, 1, 1, 256, stream, a);
}

K3H_API int k3h_moe_w_shuffle(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                              int experts, int n, int row_bytes, int gated) {
  if (!ctx || experts < 0 || n < 0 || row_bytes <= 0 || row_bytes % 16 || n % 32) return K3H_EINVAL;
  const int64_t total = (int64_t)experts * n * (row_bytes / 16);
  if (total == 0) return K3H_OK;
  if (!k3h_okp(src, 16) || !k3h_okp(dst, 16)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(src).ptr(dst).i32(experts).i32(n).i32(row_bytes).i32(gated);
  return k3h_run(ctx, kMoeV4, "kern_k3_moe_w_shuffle", k3h_cdiv(total, 256), 1, 1, 256, stream, a);
}

K3H_API int k3h_moe_sf_shuffle(k3h_ctx_t ctx, void* stream, const void* src, void* dst,
                               int experts, int n, int kg, int gated) {
  if (!ctx || experts < 0 || n < 0 || kg <= 0 || kg % 4 || n % 128) return K3H_EINVAL;
  const int64_t total = (int64_t)experts * n * kg;
  if (total == 0) return K3H_OK;
  if (!k3h_okp(src, 1) || !k3h_okp(dst, 1)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(src).ptr(dst).i32(experts).i32(n).i32(kg).i32(gated);
  return k3h_run(ctx, kMoeV4, "kern_k3_moe_sf_shuffle", k3h_cdiv(total, 256), 1, 1, 256, stream, a);
}

}  // extern "C"
