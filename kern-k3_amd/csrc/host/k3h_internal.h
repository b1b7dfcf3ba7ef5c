// Internal helpers of the k3h host library: argument packing at the kernel
// parameter buffer's natural alignment, launch through a context, and the
// host-side validation shared by the typed operator wrappers.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>

#include "k3h.h"

int k3h_hip(hipError_t e);

// Packs kernel arguments the way the manifest describes them: each argument at
// its natural alignment (8 bytes for pointers and i64, 4 for i32 and f32).
class K3hArgs {
 public:
  K3hArgs& ptr(const void* p) { return put(&p, sizeof(p), 8); }
  K3hArgs& i32(int32_t v) { return put(&v, 4, 4); }
  K3hArgs& i64(int64_t v) { return put(&v, 8, 8); }
  K3hArgs& f32(float v) { return put(&v, 4, 4); }
  const void* data() const { return buf_; }
  size_t size() const { return n_; }
  bool ok() const { return ok_; }

 private:
  K3hArgs& put(const void* p, size_t sz, size_t al) {
    n_ = (n_ + al - 1) & ~(al - 1);
    if (n_ + sz > sizeof(buf_)) { ok_ = false; return *this; }
    std::memcpy(buf_ + n_, p, sz);
    n_ += sz;
    return *this;
  }
  alignas(8) unsigned char buf_[512] = {};
  size_t n_ = 0;
  bool ok_ = true;
};

// Workgroups of `block` threads of (module, entry) that the current device holds
// at once (occupancy per CU x CUs), cached in the context.
int k3h_ctx_resident(k3h_ctx_t ctx, const char* module_key, const char* entry, uint32_t block,
                     int* out);

// Look up (module, entry) in the context and launch with packed args.
int k3h_run(k3h_ctx_t ctx, const char* module_key, const char* entry, uint32_t gx, uint32_t gy,
            uint32_t gz, uint32_t block, void* stream, const K3hArgs& a, uint32_t shmem = 0);

// K1 row bodies: the typed nb and push entries run the 256-thread vector-split
// form (k3h_land_add_attnres_rms_nb{K}s, k3h_attnres_rms_push_nb{K}s) for
// 1 <= nb <= kSplitNbMax, which covers every nb the row body takes.
constexpr int kSplitNbMax = 8;
constexpr uint32_t kSplitThreads = 256;

inline bool k3h_aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
// Non-null and `a`-byte aligned.
inline bool k3h_okp(const void* p, size_t a) { return p != nullptr && k3h_aligned(p, a); }
inline uint32_t k3h_cdiv(int64_t a, int64_t b) { return (uint32_t)((a + b - 1) / b); }
