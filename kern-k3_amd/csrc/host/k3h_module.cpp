// k3h module layer and context: hipModule loading of gfx950 code objects, entry
// lookup and packed-argument launches (the role the kern runtime's cubin
// loader plays for the reference, README.md:92-97).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <tuple>
#include <utility>

#include "k3h.h"
#include "k3h_internal.h"

struct k3h_module_s {
  hipModule_t mod;
};

int k3h_hip(hipError_t e) { return e == hipSuccess ? K3H_OK : K3H_EHIP_BASE - (int)e; }

extern "C" {

K3H_API int k3h_module_load(const void* image, size_t bytes, k3h_module_t* out) {
  if (!image || !bytes || !out) return K3H_EINVAL;
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess) return k3h_hip(e);
  k3h_module_s* h = new (std::nothrow) k3h_module_s{m};
  if (!h) { (void)hipModuleUnload(m); return K3H_ENOMEM; }
  *out = h;
  return K3H_OK;
}

K3H_API int k3h_module_load_file(const char* path, k3h_module_t* out) {
  if (!path || !out) return K3H_EINVAL;
  FILE* f = std::fopen(path, "rb");
  if (!f) return K3H_ENOMODULE;
  std::fclose(f);
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoad(&m, path);
  if (e != hipSuccess) return k3h_hip(e);
  k3h_module_s* h = new (std::nothrow) k3h_module_s{m};
  if (!h) { (void)hipModuleUnload(m); return K3H_ENOMEM; }
  *out = h;
  return K3H_OK;
}

K3H_API int k3h_function(k3h_module_t mod, const char* entry, k3h_fn_t* out) {
  if (!mod || !entry || !out) return K3H_EINVAL;
  hipFunction_t f = nullptr;
  const hipError_t e = hipModuleGetFunction(&f, mod->mod, entry);
  if (e == hipErrorNotFound) return K3H_ENOENTRY;
  if (e != hipSuccess) return k3h_hip(e);
  *out = reinterpret_cast<k3h_fn_t>(f);
  return K3H_OK;
}

K3H_API int k3h_launch(k3h_fn_t fn, const uint32_t grid[3], const uint32_t block[3],
                       uint32_t shmem, void* stream, const void* packed_args, size_t bytes) {
  if (!fn || !grid || !block) return K3H_EINVAL;
  if (bytes && !packed_args) return K3H_EINVAL;
  if (!block[0] || !block[1] || !block[2] || (uint64_t)block[0] * block[1] * block[2] > 1024)
    return K3H_EINVAL;
  if (!grid[0] || !grid[1] || !grid[2]) return K3H_OK;  // an empty grid launches nothing
  size_t size = bytes;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(packed_args),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  const hipError_t e = hipModuleLaunchKernel(
      reinterpret_cast<hipFunction_t>(fn), grid[0], grid[1], grid[2], block[0], block[1],
      block[2], shmem, static_cast<hipStream_t>(stream), nullptr, bytes ? config : nullptr);
  return k3h_hip(e);
}

K3H_API int k3h_module_unload(k3h_module_t mod) {
  if (!mod) return K3H_EINVAL;
  const hipError_t e = hipModuleUnload(mod->mod);
  delete mod;
  return k3h_hip(e);
}

K3H_API const char* k3h_error_string(int code) {
  switch (code) {
    case K3H_OK: return "ok";
    case K3H_EINVAL: return "invalid argument";
    case K3H_ENOMODULE: return "code object missing or not loadable";
    case K3H_ENOENTRY: return "entry not found in module";
    case K3H_ENOMEM: return "out of host memory";
    case K3H_ERESIDENT: return "grid larger than the device holds at once";
    default: break;
  }
  if (code <= K3H_EHIP_BASE) return hipGetErrorString(static_cast<hipError_t>(K3H_EHIP_BASE - code));
  return "unknown error";
}

K3H_API int k3h_runtime_version(int* version) {
  if (!version) return K3H_EINVAL;
  return k3h_hip(hipRuntimeGetVersion(version));
}

}  // extern "C"

// ---------------------------------------------------------------- context
struct k3h_ctx_s {
  std::string dir;
  std::mutex mu;
  std::map<std::string, k3h_module_t> mods;
  std::map<std::pair<std::string, std::string>, k3h_fn_t> fns;
  // (function, block size, device) -> workgroups the device holds at once
  std::map<std::tuple<k3h_fn_t, uint32_t, int>, int> resident;
};

int k3h_ctx_resident(k3h_ctx_t ctx, const char* module_key, const char* entry, uint32_t block,
                     int* out) {
  k3h_fn_t fn = nullptr;
  int r = k3h_ctx_function(ctx, module_key, entry, &fn);
  if (r != K3H_OK) return r;
  int dev = 0;
  r = k3h_hip(hipGetDevice(&dev));
  if (r != K3H_OK) return r;
  std::lock_guard<std::mutex> lock(ctx->mu);
  const auto key = std::make_tuple(fn, block, dev);
  auto it = ctx->resident.find(key);
  if (it == ctx->resident.end()) {
    int per_cu = 0, cus = 0;
    r = k3h_hip(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, reinterpret_cast<hipFunction_t>(fn), (int)block, 0));
    if (r != K3H_OK) return r;
    r = k3h_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if (r != K3H_OK) return r;
    it = ctx->resident.emplace(key, per_cu * cus).first;
  }
  *out = it->second;
  return K3H_OK;
}

extern "C" {

K3H_API int k3h_ctx_create(const char* codeobj_dir, k3h_ctx_t* out) {
  if (!codeobj_dir || !out) return K3H_EINVAL;
  k3h_ctx_s* c = new (std::nothrow) k3h_ctx_s;
  if (!c) return K3H_ENOMEM;
  c->dir = codeobj_dir;
  *out = c;
  return K3H_OK;
}

K3H_API int k3h_ctx_destroy(k3h_ctx_t ctx) {
  if (!ctx) return K3H_EINVAL;
  int rc = K3H_OK;
  for (auto& kv : ctx->mods) {
    const int r = k3h_module_unload(kv.second);
    if (r != K3H_OK) rc = r;
  }
  delete ctx;
  return rc;
}

K3H_API int k3h_ctx_function(k3h_ctx_t ctx, const char* module_key, const char* entry,
                             k3h_fn_t* out) {
  if (!ctx || !module_key || !entry || !out) return K3H_EINVAL;
  std::lock_guard<std::mutex> lock(ctx->mu);
  const auto key = std::make_pair(std::string(module_key), std::string(entry));
  auto it = ctx->fns.find(key);
  if (it != ctx->fns.end()) { *out = it->second; return K3H_OK; }
  k3h_module_t m = nullptr;
  auto mi = ctx->mods.find(key.first);
  if (mi == ctx->mods.end()) {
    const std::string path = ctx->dir + "/" + key.first + ".hsaco";
    const int r = k3h_module_load_file(path.c_str(), &m);
    if (r != K3H_OK) return r == K3H_EINVAL ? K3H_ENOMODULE : r;
    ctx->mods[key.first] = m;
  } else {
    m = mi->second;
  }
  k3h_fn_t f = nullptr;
  const int r = k3h_function(m, entry, &f);
  if (r != K3H_OK) return r;
  ctx->fns[key] = f;
  *out = f;
  return K3H_OK;
}

}  // extern "C"
