/* The C-ABI used from plain C, host side only (no GPU needed): include/k3h.h
 * compiles as C, libk3h.so links, a context opens over the built code objects,
 * and bad arguments are rejected before any HIP call.  Built and run by
 * tests/test_abi_c.py (gcc -std=c11). */
#include <stdio.h>
#include <string.h>

#include "k3h.h"

#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);        \
      return 1;                                                           \
    }                                                                     \
  } while (0)

int main(int argc, char** argv) {
  const char* dir = argc > 1 ? argv[1] : "kern-k3_amd/build";
  k3h_ctx_t ctx = NULL;
  CHECK(k3h_ctx_create(dir, &ctx) == K3H_OK && ctx != NULL);
  void* A = (void*)0x10000; /* aligned stand-in address, never dereferenced here */
  unsigned long long* F = (unsigned long long*)0x10000;
  /* fused op: negative rows, misaligned x */
  CHECK(k3h_residual_rms_mxfp8(ctx, NULL, A, A, A, A, A, A, NULL, 1e-6f, -1) == K3H_EINVAL);
  CHECK(k3h_residual_rms_mxfp8(ctx, NULL, (char*)A + 2, A, A, A, A, A, NULL, 1e-6f, 1) ==
        K3H_EINVAL);
  /* empty work is not an error and launches nothing */
  CHECK(k3h_residual_rms_mxfp8(ctx, NULL, A, A, A, A, A, A, NULL, 1e-6f, 0) == K3H_OK);
  /* MX quant: 21 elements are not whole 32-blocks */
  CHECK(k3h_moe_quant(ctx, NULL, A, A, A, 3, 7) == K3H_EINVAL);
  /* barrier: slot 0 is the epoch, 1 <= nranks <= 8, units >= 1, 8-byte counters */
  CHECK(k3h_rs_arrive(ctx, NULL, F, F, 896, 0, 4, NULL) == K3H_EINVAL);
  CHECK(k3h_rs_arrive(ctx, NULL, F, F, 896, 1, 9, NULL) == K3H_EINVAL);
  CHECK(k3h_rs_arrive(ctx, NULL, (unsigned long long*)0x10004, F, 896, 1, 4, NULL) == K3H_EINVAL);
  CHECK(k3h_epoch_bump(ctx, NULL, F, 0) == K3H_EINVAL);
  CHECK(k3h_flags_init(ctx, NULL, F, 0) == K3H_OK);
  /* null context */
  CHECK(k3h_flags_init(NULL, NULL, F, 4) == K3H_EINVAL);
  /* errors have text */
  CHECK(strlen(k3h_error_string(K3H_EINVAL)) > 0);
  CHECK(strlen(k3h_error_string(K3H_ENOENTRY)) > 0);
  CHECK(k3h_ctx_destroy(ctx) == K3H_OK);
  puts("c-abi host checks ok");
  return 0;
}
