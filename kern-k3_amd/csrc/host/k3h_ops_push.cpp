// Typed wrappers: the residual push family (res_in with the normed row stored
// into every TP rank's normed_all, its statistics hand-off to res_mlp, and the
// land_add2 fold), plus res_mlp's statistics-consuming nb entries.  One
// workgroup per row, grid ceil_div(tokens, 4) = B rows per rank as the manifest's
// (k3-tp4-prefill-16k.json:406806 attnres_rms_push_first_v3, 407299
// attnres_rms_push_add2, 406999 land_add_attnres_rms_bf16_v2_nb4): 896 threads
// at nb 0, 256 threads (the vector-split entries) at nb >= 1; the manifest's
// 128-thread entry serves the module-layer launch.
#include <string>

#include "k3h_internal.h"

namespace {

constexpr int kNbMax = 8;
constexpr int kMaxRanks = 8;
constexpr uint32_t kResThreads = 128;
constexpr uint32_t kWideThreads = 896;

// Checks shared by the push entries; dst_peer is read only for q < nranks, q != rank.
int check_push(const void* blocks, const float* sw, const void* gamma, const void* normed_all,
               const unsigned long long* dst_peer, int nb, int snapshot, int B, int rank,
               int nranks) {
  if (B < 0 || nb < 0 || nb > kNbMax || nranks < 1 || nranks > kMaxRanks || rank < 0 ||
      rank >= nranks)
    return K3H_EINVAL;
  if (!k3h_okp(gamma, 16) || !k3h_okp(normed_all, 16)) return K3H_EINVAL;
  if (nb > 0 && (!k3h_okp(blocks, 16) || !k3h_okp(sw, 16))) return K3H_EINVAL;
  if (snapshot && nb < kNbMax && !k3h_okp(blocks, 16)) return K3H_EINVAL;
  if (nranks > 1 && !k3h_okp(dst_peer, 8)) return K3H_EINVAL;
  return K3H_OK;
}

// nb == 0: the module's 896-thread entry (one 16-byte vector of the row per
// lane); 1 <= nb <= kSplitNbMax: its 256-thread vector-split entry for that nb;
// otherwise the 128-thread manifest entry.  Same parameter list and outputs.
struct PushEntry {
  std::string name;
  uint32_t threads;
};
PushEntry push_entry(int nb) {
  if (nb == 0) return {"k3h_attnres_rms_push_nb0w896", kWideThreads};
  if (nb >= 1 && nb <= kSplitNbMax)
    return {"k3h_attnres_rms_push_nb" + std::to_string(nb) + "s", kSplitThreads};
  return {"kern_k3_attnres_rms_push", kResThreads};
}

void push_common(K3hArgs& a, void* blocks, const float* sw, const void* gamma, void* normed_all,
                 const unsigned long long* dst_peer, int nb, int snapshot, int B, int rank,
                 int nranks) {
  a.ptr(blocks).ptr(sw).ptr(gamma).ptr(normed_all).ptr(dst_peer);
  a.i32(nb).i32(snapshot).i32(B).i32(rank).i32(nranks);
}

}  // namespace

extern "C" {

K3H_API int k3h_attnres_rms_push(k3h_ctx_t ctx, void* stream, int version, const void* prefix,
                                 void* blocks, const float* sw, const void* gamma,
                                 void* normed_all, const unsigned long long* dst_peer, int nb,
                                 int snapshot, int B, int rank, int nranks) {
  if (!ctx || (version != 1 && version != 3)) return K3H_EINVAL;
  const int r = check_push(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  if (r != K3H_OK) return r;
  if (!k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(prefix);
  push_common(a, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  const PushEntry e = push_entry(nb);
  return k3h_run(ctx, version == 1 ? "k3_residual_push" : "k3_residual_push_v3", e.name.c_str(),
                 (uint32_t)B, 1, 1, e.threads, stream, a);
}

K3H_API int k3h_attnres_rms_push_stats(k3h_ctx_t ctx, void* stream, const void* prefix,
                                       void* blocks, const float* sw, const void* gamma,
                                       void* normed_all, const unsigned long long* dst_peer,
                                       int nb, int snapshot, int B, int rank, int nranks,
                                       const float* sw_mlp, float* stats) {
  if (!ctx) return K3H_EINVAL;
  const int r = check_push(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  if (r != K3H_OK) return r;
  if (!k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (nb > 0 && (!k3h_okp(sw_mlp, 16) || !k3h_okp(stats, 8))) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(prefix);
  push_common(a, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  a.ptr(sw_mlp).ptr(stats);
  const PushEntry e = push_entry(nb);
  return k3h_run(ctx, "k3_residual_push_stats", e.name.c_str(), (uint32_t)B, 1, 1, e.threads,
                 stream, a);
}

K3H_API int k3h_attnres_rms_push_add2(k3h_ctx_t ctx, void* stream, void* blocks, const float* sw,
                                      const void* gamma, void* normed_all,
                                      const unsigned long long* dst_peer, int nb, int snapshot,
                                      int B, int rank, int nranks, const float* sw_mlp,
                                      float* stats, const void* p1, const void* p2,
                                      const void* prefix2, void* hidden, int two) {
  if (!ctx) return K3H_EINVAL;
  const int r = check_push(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  if (r != K3H_OK) return r;
  if (nb > 0 && (!k3h_okp(sw_mlp, 16) || !k3h_okp(stats, 8))) return K3H_EINVAL;
  if (!k3h_okp(p1, 16) || !k3h_okp(prefix2, 16) || !k3h_okp(hidden, 16)) return K3H_EINVAL;
  if (two && !k3h_okp(p2, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  push_common(a, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks);
  a.ptr(sw_mlp).ptr(stats).ptr(p1).ptr(p2).ptr(prefix2).ptr(hidden).i32(two);
  const PushEntry e = push_entry(nb);
  return k3h_run(ctx, "k3_residual_push_add2", e.name.c_str(), (uint32_t)B, 1, 1, e.threads,
                 stream, a);
}

K3H_API int k3h_land_add_attnres_rms_nb_stats(k3h_ctx_t ctx, void* stream, const void* partial,
                                              const void* prefix, const void* blocks,
                                              const float* sw, const void* gamma, void* prefix2,
                                              void* normed, int nb, int snapshot, int B,
                                              const float* stats, int nb_stats) {
  if (!ctx || B < 0 || nb < 1 || nb > kNbMax || nb_stats < 0 || nb_stats > nb) return K3H_EINVAL;
  if (!k3h_okp(gamma, 16) || !k3h_okp(normed, 16) || !k3h_okp(blocks, 16) || !k3h_okp(sw, 16))
    return K3H_EINVAL;
  if (!k3h_okp(partial, 16) || !k3h_okp(prefix2, 16)) return K3H_EINVAL;
  if (!snapshot && !k3h_okp(prefix, 16)) return K3H_EINVAL;
  if (nb_stats > 0 && !k3h_okp(stats, 8)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  const bool split = nb <= kSplitNbMax;
  const std::string entry = (split ? "k3h_land_add_attnres_rms_nb" : "kern_k3_land_add_attnres_rms_nb") +
                            std::to_string(nb) + (split ? "s" : "");
  K3hArgs a;
  a.ptr(partial).ptr(prefix).ptr(blocks).ptr(sw).ptr(gamma).ptr(prefix2).ptr(normed);
  a.i32(nb).i32(snapshot).i32(B).ptr(stats).i32(nb_stats);
  return k3h_run(ctx, "k3_residual_nb_stats", entry.c_str(), (uint32_t)B, 1, 1,
                 split ? kSplitThreads : kResThreads, stream, a);
}

K3H_API int k3h_land_add2_bf16(k3h_ctx_t ctx, void* stream, const void* p1, const void* p2,
                               const void* prefix2, void* hidden, int two, int B) {
  if (!ctx || B < 0) return K3H_EINVAL;
  if (!k3h_okp(p1, 16) || !k3h_okp(prefix2, 16) || !k3h_okp(hidden, 16)) return K3H_EINVAL;
  if (two && !k3h_okp(p2, 16)) return K3H_EINVAL;
  if (B == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(p1).ptr(p2).ptr(prefix2).ptr(hidden).i32(two).i32(B);
  return k3h_run(ctx, "k3_land_bf16", "kern_k3_land_add2_bf16", (uint32_t)B, 1, 1, kResThreads,
                 stream, a);
}

// ---- epoch / arrival barrier (module k3_barrier.hip) -----------------------

K3H_API int k3h_flags_init(k3h_ctx_t ctx, void* stream, unsigned long long* flags, int n) {
  if (!ctx || n < 0 || !k3h_okp(flags, 8)) return K3H_EINVAL;
  if (n == 0) return K3H_OK;
  K3hArgs a;
  a.ptr(flags).i32(n);
  return k3h_run(ctx, "k3_collectives", "kern_k3_flags_init", 1, 1, 1, 256, stream, a);
}

// kern_k3_epoch_bump adds its grid size; one 64-thread workgroup per unit (the
// reference's 1024-thread workgroups add the same count).
K3H_API int k3h_epoch_bump(k3h_ctx_t ctx, void* stream, unsigned long long* flags, int units) {
  if (!ctx || units < 1 || !k3h_okp(flags, 8)) return K3H_EINVAL;
  K3hArgs a;
  a.ptr(flags);
  return k3h_run(ctx, "k3_collectives", "kern_k3_epoch_bump", (uint32_t)units, 1, 1, 64, stream,
                 a);
}

K3H_API int k3h_rs_arrive(k3h_ctx_t ctx, void* stream, unsigned long long* flags,
                          const unsigned long long* flags_peer, int units, int slot, int nranks,
                          unsigned* missing) {
  if (!ctx || units < 1 || slot < 1 || nranks < 1 || nranks > kMaxRanks) return K3H_EINVAL;
  if (!k3h_okp(flags, 8) || !k3h_okp(flags_peer, 8)) return K3H_EINVAL;
  if (missing && !k3h_okp(missing, 4)) return K3H_EINVAL;
  K3hArgs a;
  if (!missing) {  // the manifest entry (src, dst, src_peer, count, order, rank unused)
    a.ptr(nullptr).ptr(nullptr).ptr(nullptr).ptr(flags).ptr(flags_peer).i64(0);
    a.i32(units).i32(slot).i32(6).i32(0).i32(nranks);
    return k3h_run(ctx, "k3_rs_arrive_v2", "kern_k3_rs_arrive1", 1, 1, 1, 64, stream, a);
  }
  a.ptr(flags).ptr(flags_peer).i32(units).i32(slot).i32(nranks).ptr(missing);
  return k3h_run(ctx, "k3_rs_arrive_v2", "k3h_rs_arrive_mask", 1, 1, 1, 64, stream, a);
}

}  // extern "C"
