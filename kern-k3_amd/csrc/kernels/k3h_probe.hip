// Module k3h_probe: measurement kernels, not operators.  They set the ceilings
// the operators' rates are read against: what HBM delivers for a given access
// shape (read only, write only, copy, and the fused op's 2 reads : 1.5 writes),
// with several loads in flight per lane and with a persistent grid, and the
// issue rate of the MX-scaled matrix-core instruction the MoE GEMMs use.
//
// Streaming probes (block 256; n16 = 16-byte vectors per stream):
//   k3h_probe_<op>_u<U>     grid n16 / (256 U): workgroup w moves vectors
//                           [256 U w, 256 U (w + 1)), U coalesced 4 KB rows of
//                           the block, all U loads issued before any use
//   k3h_probe_<op>_u<U>p    persistent: any grid; workgroups stride over those
//                           256 U-vector blocks
//   <op> = read   (src -> xor into one word, stored only if it equals a value
//                  no input here produces, so the loads stay live)
//          write  (a constant -> dst)
//          copy   (src -> dst)
//          shape  (a, b -> c (16 B) and d (8 B) per vector: the byte shape of
//                  the fused residual + RMSNorm + MXFP8 op, 2 reads : 1.5 writes)
//   suffix _c: cacheable loads and stores instead of non-temporal ones.
//   The host keeps n16 a multiple of 256 U (no bounds checks in the loops).
//
// MFMA probe: k3h_probe_mfma_<A><B>(out, iters), block 256, any grid: each
// wave issues iters x 4 independent v_mfma_scale_f32_32x32x64_f8f6f4 on
// register operands (A format e4m3 "f8" or e2m1 "f4", likewise B; unit scales);
// one instruction is 32 x 32 x 64 x 2 = 131072 FLOPs.  Lane sums go to
// out[global thread id].
#include "../common/k3_dev.h"

typedef int k3_v8i __attribute__((ext_vector_type(8)));
typedef float k3_v16f __attribute__((ext_vector_type(16)));

template <bool NT>
K3_DEV k3_u4 kp_ld(const k3_u4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT>
K3_DEV void kp_st(k3_u4* p, k3_u4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}
template <bool NT>
K3_DEV void kp_st8(k3_u2* p, k3_u2 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Block loop: flat grids take their one block, persistent grids stride.
#define KP_BLOCKS(U, P)                                                            \
  for (long long blk = blockIdx.x; blk * 256 * (U) < n16; blk += (P) ? gridDim.x : n16)

template <int U, bool P, bool NT>
K3_DEV void kp_read(const k3_u4* __restrict__ src, long long n16, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  KP_BLOCKS(U, P) {
    const k3_u4* s = src + blk * 256 * U + threadIdx.x;
    k3_u4 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) v[k] = kp_ld<NT>(s + 256 * k);
#pragma unroll
    for (int k = 0; k < U; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;  // never true for the probe's inputs
}

template <int U, bool P, bool NT>
K3_DEV void kp_write(k3_u4* __restrict__ dst, long long n16, uint32_t val) {
  const k3_u4 v = {val, val, val, val};
  KP_BLOCKS(U, P) {
    k3_u4* d = dst + blk * 256 * U + threadIdx.x;
#pragma unroll
    for (int k = 0; k < U; ++k) kp_st<NT>(d + 256 * k, v);
  }
}

template <int U, bool P, bool NT>
K3_DEV void kp_copy(const k3_u4* __restrict__ src, k3_u4* __restrict__ dst, long long n16) {
  KP_BLOCKS(U, P) {
    const long long o = blk * 256 * U + threadIdx.x;
    k3_u4 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) v[k] = kp_ld<NT>(src + o + 256 * k);
#pragma unroll
    for (int k = 0; k < U; ++k) kp_st<NT>(dst + o + 256 * k, v[k]);
  }
}

template <int U, bool P, bool NT>
K3_DEV void kp_shape(const k3_u4* __restrict__ a, const k3_u4* __restrict__ b,
                     k3_u4* __restrict__ c, k3_u2* __restrict__ d, long long n16) {
  KP_BLOCKS(U, P) {
    const long long o = blk * 256 * U + threadIdx.x;
    k3_u4 va[U], vb[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      va[k] = kp_ld<NT>(a + o + 256 * k);
      vb[k] = kp_ld<NT>(b + o + 256 * k);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const k3_u4 s = va[k] ^ vb[k];
      kp_st<NT>(c + o + 256 * k, s);
      kp_st8<NT>(d + o + 256 * k, (k3_u2){s[0] ^ s[1], s[2] ^ s[3]});
    }
  }
}

#define KP_ENTRIES(SUF, U, P, NT)                                                             \
  extern "C" __global__ void __launch_bounds__(256)                                           \
      k3h_probe_read_##SUF(const k3_u4* src, long long n16, uint32_t* sink) {                 \
    kp_read<U, P, NT>(src, n16, sink);                                                        \
  }                                                                                           \
  extern "C" __global__ void __launch_bounds__(256)                                           \
      k3h_probe_write_##SUF(k3_u4* dst, long long n16, uint32_t val) {                        \
    kp_write<U, P, NT>(dst, n16, val);                                                        \
  }                                                                                           \
  extern "C" __global__ void __launch_bounds__(256)                                           \
      k3h_probe_copy_##SUF(const k3_u4* src, k3_u4* dst, long long n16) {                     \
    kp_copy<U, P, NT>(src, dst, n16);                                                         \
  }                                                                                           \
  extern "C" __global__ void __launch_bounds__(256) k3h_probe_shape_##SUF(                    \
      const k3_u4* a, const k3_u4* b, k3_u4* c, k3_u2* d, long long n16) {                    \
    kp_shape<U, P, NT>(a, b, c, d, n16);                                                      \
  }

KP_ENTRIES(u1, 1, false, true)
KP_ENTRIES(u2, 2, false, true)
KP_ENTRIES(u4, 4, false, true)
KP_ENTRIES(u7, 7, false, true)
KP_ENTRIES(u8, 8, false, true)
KP_ENTRIES(u4p, 4, true, true)
KP_ENTRIES(u8p, 8, true, true)
KP_ENTRIES(u4_c, 4, false, false)

// ---------------------------------------------------------------- MFMA rate
template <int FA, int FB>
K3_DEV void kp_mfma(float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  // operand bits: small finite codes of either format (fp4 nibbles 0x1-0x7,
  // e4m3 bytes 0x38-0x3f), varied by lane so no operand is all zeros
  const int pa = FA == 4 ? 0x13571357 + lane : 0x383a3c3e + lane;
  const int pb = FB == 4 ? 0x24672467 + lane : 0x393b3d3f + lane;
  const k3_v8i av = {pa, pa + 1, pa + 2, pa + 3, pa + 4, pa + 5, pa + 6, pa + 7};
  const k3_v8i bv = {pb, pb + 1, pb + 2, pb + 3, pb + 4, pb + 5, pb + 6, pb + 7};
  k3_v16f acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[c][q] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc[c], FA, FB, 0, 127, 0,
                                                                127);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int q = 0; q < 16; ++q) s += acc[c][q];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

extern "C" __global__ void __launch_bounds__(256) k3h_probe_mfma_f8f4(float* out, int iters) {
  kp_mfma<0, 4>(out, iters);
}
extern "C" __global__ void __launch_bounds__(256) k3h_probe_mfma_f8f8(float* out, int iters) {
  kp_mfma<0, 0>(out, iters);
}
extern "C" __global__ void __launch_bounds__(256) k3h_probe_mfma_f4f4(float* out, int iters) {
  kp_mfma<4, 4>(out, iters);
}
