/* The C-ABI from a plain C host on the GPU: no Python, no torch.  Device memory
 * comes from the HIP runtime's C API; the program runs
 *   1. the typed call k3h_residual_rms_mxfp8 (config 2's op) on 67 rows, an odd
 *      count, so the last workgroup's second row lies past B, and
 *   2. the manifest path a kern runtime takes for a code object:
 *      k3h_module_load_file / k3h_function / k3h_launch of kern_k3_moe_quant
 *      with the manifest op moe_quant's packed arguments (x, q, sf, rows, 3584)
 *      and grid ceil(ceil(tokens / 4) * 112 / 256) x 256 threads, tokens being
 *      the chunk's token count and rows = tokens / 4 this rank's share
 *      (k3-tp4-prefill-16k.json op moe_quant),
 * and compares every output byte for byte with the C oracle (test
 * infrastructure: the checker, not the measured path).  Outputs are filled
 * with 0xA5 first, so a byte the kernels never wrote shows as a mismatch.
 * Built and run by tests/test_abi_c.py; exit status 77 when no device is
 * visible. */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "k3_oracle.h"
#include "k3h.h"

#define H 7168

#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);        \
      return 1;                                                           \
    }                                                                     \
  } while (0)

#define HIPCHECK(x)                                                               \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
              __LINE__);                                                          \
      return 1;                                                                   \
    }                                                                             \
  } while (0)

static uint64_t g_state = 0x9E3779B97F4A7C15ull;

static double uniform01(void) {  // xorshift64*
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return (double)((g_state * 0x2545F4914F6CDD1Dull) >> 11) * 0x1.0p-53;
}

// bf16 values uniform in [-scale, scale), one in a thousand times 50
static int fill_bf16(uint16_t* y, size_t n, float scale) {
  float* f = (float*)malloc(n * sizeof(float));
  if (!f) return 1;
  for (size_t i = 0; i < n; ++i) {
    f[i] = (float)((uniform01() * 2.0 - 1.0) * scale);
    if (uniform01() < 0.001) f[i] *= 50.0f;
  }
  k3o_f2bf_n(f, y, n);
  free(f);
  return 0;
}

// 0 when equal, else prints the first differing byte and returns 1
static int compare(const char* what, const void* got, const void* want, size_t bytes) {
  const unsigned char* g = (const unsigned char*)got;
  const unsigned char* w = (const unsigned char*)want;
  for (size_t i = 0; i < bytes; ++i)
    if (g[i] != w[i]) {
      fprintf(stderr, "FAIL %s: byte %zu of %zu: got 0x%02x, oracle 0x%02x\n", what, i, bytes,
              g[i], w[i]);
      return 1;
    }
  printf("%s: %zu bytes equal to the oracle\n", what, bytes);
  return 0;
}

static int fused_case(k3h_ctx_t ctx, hipStream_t st) {
  const int B = 67;
  const size_t n = (size_t)B * H;
  uint16_t *x = malloc(n * 2), *r = malloc(n * 2), *g = malloc(H * 2);
  uint16_t *ro = malloc(n * 2), *nm = malloc(n * 2), *ro_o = malloc(n * 2), *nm_o = malloc(n * 2);
  uint8_t *q = malloc(n), *sf = malloc(n / 32), *q_o = malloc(n), *sf_o = malloc(n / 32);
  CHECK(x && r && g && ro && nm && ro_o && nm_o && q && sf && q_o && sf_o);
  CHECK(fill_bf16(x, n, 1.0f) == 0 && fill_bf16(r, n, 2.0f) == 0 && fill_bf16(g, H, 1.0f) == 0);

  void *dx, *dr, *dg, *dro, *dq, *dsf, *dnm;
  HIPCHECK(hipMalloc(&dx, n * 2));
  HIPCHECK(hipMalloc(&dr, n * 2));
  HIPCHECK(hipMalloc(&dg, H * 2));
  HIPCHECK(hipMalloc(&dro, n * 2));
  HIPCHECK(hipMalloc(&dq, n));
  HIPCHECK(hipMalloc(&dsf, n / 32));
  HIPCHECK(hipMalloc(&dnm, n * 2));
  HIPCHECK(hipMemcpy(dx, x, n * 2, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(dr, r, n * 2, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(dg, g, H * 2, hipMemcpyHostToDevice));
  HIPCHECK(hipMemset(dro, 0xA5, n * 2));
  HIPCHECK(hipMemset(dq, 0xA5, n));
  HIPCHECK(hipMemset(dsf, 0xA5, n / 32));
  HIPCHECK(hipMemset(dnm, 0xA5, n * 2));

  printf("[case] typed call k3h_residual_rms_mxfp8, B %d, eps 1e-6\n", B);
  fflush(stdout);
  CHECK(k3h_residual_rms_mxfp8(ctx, st, dx, dr, dg, dro, dq, dsf, dnm, 1e-6f, B) == K3H_OK);
  HIPCHECK(hipStreamSynchronize(st));
  HIPCHECK(hipMemcpy(ro, dro, n * 2, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(q, dq, n, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(sf, dsf, n / 32, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(nm, dnm, n * 2, hipMemcpyDeviceToHost));

  k3o_residual_rms_mxfp8(x, r, g, ro_o, q_o, sf_o, nm_o, B, 1e-6f);
  int bad = compare("residual_out", ro, ro_o, n * 2) | compare("q (e4m3)", q, q_o, n) |
            compare("sf (E8M0)", sf, sf_o, n / 32) | compare("normed", nm, nm_o, n * 2);

  HIPCHECK(hipFree(dx));
  HIPCHECK(hipFree(dr));
  HIPCHECK(hipFree(dg));
  HIPCHECK(hipFree(dro));
  HIPCHECK(hipFree(dq));
  HIPCHECK(hipFree(dsf));
  HIPCHECK(hipFree(dnm));
  free(x); free(r); free(g); free(ro); free(nm); free(ro_o); free(nm_o);
  free(q); free(sf); free(q_o); free(sf_o);
  return bad;
}

static int manifest_case(const char* dir, hipStream_t st) {
  const int T = 37, cols = 3584;
  const size_t n = (size_t)T * cols;
  uint16_t* x = malloc(n * 2);
  uint8_t *q = malloc(n), *sf = malloc(n / 32), *q_o = malloc(n), *sf_o = malloc(n / 32);
  CHECK(x && q && sf && q_o && sf_o);
  CHECK(fill_bf16(x, n, 3.0f) == 0);

  void *dx, *dq, *dsf;
  HIPCHECK(hipMalloc(&dx, n * 2));
  HIPCHECK(hipMalloc(&dq, n));
  HIPCHECK(hipMalloc(&dsf, n / 32));
  HIPCHECK(hipMemcpy(dx, x, n * 2, hipMemcpyHostToDevice));
  HIPCHECK(hipMemset(dq, 0xA5, n));
  HIPCHECK(hipMemset(dsf, 0xA5, n / 32));

  char path[4096];
  snprintf(path, sizeof path, "%s/%s.hsaco", dir, "k3_moe_prefill_v3+EP_STRIDED=1");
  k3h_module_t mod = NULL;
  k3h_fn_t fn = NULL;
  CHECK(k3h_module_load_file(path, &mod) == K3H_OK);
  CHECK(k3h_function(mod, "kern_k3_moe_quant", &fn) == K3H_OK);
  CHECK(k3h_function(mod, "kern_k3_no_such_entry", &fn) == K3H_ENOENTRY);
  CHECK(k3h_function(mod, "kern_k3_moe_quant", &fn) == K3H_OK);

  // the manifest op's launch: args (param 0, 1, 2, 3, i32 3584), natural alignment
  unsigned char args[32];
  memset(args, 0, sizeof args);
  memcpy(args + 0, &dx, 8);
  memcpy(args + 8, &dq, 8);
  memcpy(args + 16, &dsf, 8);
  memcpy(args + 24, &T, 4);
  memcpy(args + 28, &cols, 4);
  const int tokens = 4 * T;  // the manifest's grid variable: the chunk's tokens
  const uint32_t grid[3] = {(uint32_t)(((tokens + 3) / 4 * 112 + 255) / 256), 1, 1};
  const uint32_t block[3] = {256, 1, 1};
  printf("[case] manifest op moe_quant through k3h_launch, rows %d, grid %u\n", T, grid[0]);
  fflush(stdout);
  CHECK(k3h_launch(fn, grid, block, 0, st, args, sizeof args) == K3H_OK);
  HIPCHECK(hipStreamSynchronize(st));
  HIPCHECK(hipMemcpy(q, dq, n, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(sf, dsf, n / 32, hipMemcpyDeviceToHost));
  CHECK(k3h_module_unload(mod) == K3H_OK);

  k3o_moe_quant(x, q_o, sf_o, T, cols);
  int bad = compare("moe_quant q", q, q_o, n) | compare("moe_quant sf", sf, sf_o, n / 32);

  HIPCHECK(hipFree(dx));
  HIPCHECK(hipFree(dq));
  HIPCHECK(hipFree(dsf));
  free(x); free(q); free(sf); free(q_o); free(sf_o);
  return bad;
}

int main(int argc, char** argv) {
  const char* dir = argc > 1 ? argv[1] : "kern-k3_amd/build";
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    printf("no HIP device visible\n");
    return 77;
  }
  HIPCHECK(hipSetDevice(0));
  int version = 0;
  CHECK(k3h_runtime_version(&version) == K3H_OK && version > 0);
  k3h_ctx_t ctx = NULL;
  CHECK(k3h_ctx_create(dir, &ctx) == K3H_OK);
  hipStream_t st;
  HIPCHECK(hipStreamCreate(&st));
  int bad = fused_case(ctx, st) | manifest_case(dir, st);
  HIPCHECK(hipStreamDestroy(st));
  CHECK(k3h_ctx_destroy(ctx) == K3H_OK);
  if (bad) return 1;
  printf("c-abi gpu parity ok\n");
  return 0;
}
