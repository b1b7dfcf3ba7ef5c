// Modules k3_quant_fp8_pair / k3_quant_fp8_pair_v2: per-tensor bf16 -> e4m3.
//
//   v1: kern_quant_fp8_amax(x, n, partials)                   (k3_quant_fp8_pair.cu:18)
//       kern_quant_fp8_apply(x, y, n, partials, nb, scale_out) (k3_quant_fp8_pair.cu:32)
//   v2: kern_quant_fp8_amax_v2 / kern_quant_fp8_apply_v2 with the same
//       parameters (k3_quant_fp8_pair_v2.cu:42, 63; manifest op quant_fp8_tensor,
//       k3-tp4-prefill-16k.json:407194)
//   grid (nb, 1, 1) with nb = 2048 in the manifest, block (256, 1, 1), both launches.
//
// amax:  partials[b] = max |x| over block b's slice of a grid-stride partition.
//        v1 partitions elements (element i belongs to block (i / 256) % nb) and
//        takes an f32 max (NaN ignored); v2 partitions 16-byte vectors (vector i
//        to block (i / 256) % nb), takes the max of the |bf16| bit patterns
//        (NaN patterns included) and folds the n % 8 tail into block 0.  The
//        partials are outputs, so the slices follow those partitions exactly;
//        only the order inside a slice is free (the max is order-independent).
// apply: amax = max(partials[0..nb)), scale = amax > 0 ? amax / 448 : 1 (IEEE
//        division), scale_out[0] = scale, y = e4m3(x * (1 / scale)) with RNE and
//        saturation to +-448.  |x| * (1 / scale) exceeds 448 by rounding only,
//        which the RNE conversion maps back to 448.
// Cache policy: the amax pass reads x with cacheable loads, so that x (235 MB
// at 16384 x 7168) stays in the 256 MB MALL and the apply pass, which sweeps
// it in the same front-to-back order, reads it from there; the apply pass's
// own loads and stores are non-temporal (measured at that shape: 99.4 -> 90.5
// us after a clean 512 MB flush, 96.0 -> 87.8 us back to back over four
// rotating input / output sets, identical outputs; after a dirty 512 MB flush
// the amax pass pays the write-back of the lines it evicts, 97 -> 131 us).
#include "../common/k3_dev.h"

#define QT 256

// Block max of a non-negative u32 (four waves: wave butterfly, then LDS).
K3_DEV uint32_t k3_block_max_u32(uint32_t m) {
  __shared__ uint32_t s[QT / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t p = (uint32_t)__shfl_xor((int)m, o, 64);
    m = m > p ? m : p;
  }
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
  __syncthreads();
  uint32_t r = s[0];
#pragma unroll
  for (int w = 1; w < QT / 64; ++w) r = r > s[w] ? r : s[w];
  return r;
}

// |bf16| magnitude key for the f32-max form: NaN patterns are ignored (0).
K3_DEV uint32_t k3_mag_f32max(uint32_t h) {
  const uint32_t a = h & 0x7fffu;
  return a > 0x7f80u ? 0u : a;
}

#ifndef K3_QUANT_V2
extern "C" __global__ void __launch_bounds__(QT) kern_quant_fp8_amax(
    const uint16_t* __restrict__ x, int n, float* __restrict__ partials) {
  // block b owns the 256-element chunks b, b + nb, b + 2 nb, ...; a 256-thread
  // step covers eight chunks with one 16-byte vector per thread (32 per chunk).
  const long long nb = gridDim.x;
  const int sub = threadIdx.x >> 5, lane = threadIdx.x & 31;
  uint32_t m = 0;
  for (long long c = blockIdx.x + sub * nb; c * 256 < n; c += 8 * nb) {
    const long long e0 = c * 256 + lane * 8;
    if (e0 + 8 <= n) {
      const k3_u4 v = k3_ld16(x + e0);  // cacheable: kept in the MALL for the apply pass
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = k3_mag_f32max(v[j] & 0xffffu), hi = k3_mag_f32max(v[j] >> 16);
        m = m > lo ? m : lo;
        m = m > hi ? m : hi;
      }
    } else {
      for (long long e = e0; e < n; ++e) {
        const uint32_t a = k3_mag_f32max(x[e]);
        m = m > a ? m : a;
      }
    }
  }
  m = k3_block_max_u32(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = __uint_as_float(m << 16);
}
#define K3_APPLY_NAME kern_quant_fp8_apply
#else
extern "C" __global__ void __launch_bounds__(QT) kern_quant_fp8_amax_v2(
    const uint16_t* __restrict__ x, int n, float* __restrict__ partials) {
  const long long nv = n >> 3;
  uint32_t m = 0;
  for (long long i = (long long)blockIdx.x * QT + threadIdx.x; i < nv; i += (long long)gridDim.x * QT) {
    const k3_u4 v = k3_ld16(x + i * 8);  // cacheable: kept in the MALL for the apply pass
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = v[j] & 0x7fff7fffu;
      const uint32_t lo = a & 0xffffu, hi = a >> 16;
      m = m > lo ? m : lo;
      m = m > hi ? m : hi;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const uint32_t a = x[nv * 8 + threadIdx.x] & 0x7fffu;
    m = m > a ? m : a;
  }
  m = k3_block_max_u32(m);
  if (threadIdx.x == 0) partials[blockIdx.x] = __uint_as_float(m << 16);
}
#define K3_APPLY_NAME kern_quant_fp8_apply_v2
#endif

extern "C" __global__ void __launch_bounds__(QT) K3_APPLY_NAME(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ y, int n,
    const float* __restrict__ partials, int nb, float* __restrict__ scale_out) {
  __shared__ float s[QT / 64];
  float m = 0.0f;
  for (int b = threadIdx.x; b < nb; b += QT) m = fmaxf(m, partials[b]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
  __syncthreads();
  float amax = s[0];
#pragma unroll
  for (int w = 1; w < QT / 64; ++w) amax = fmaxf(amax, s[w]);
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  if (blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
  const float inv = 1.0f / scale;

  const long long nv = n >> 3;
  for (long long i = (long long)blockIdx.x * QT + threadIdx.x; i < nv; i += (long long)gridDim.x * QT) {
    const k3_u4 v = k3_ld16_nt(x + i * 8);
    k3_u2 o;
    o[0] = k3_pack_e4m3x4(k3_bf_lo(v[0]) * inv, k3_bf_hi(v[0]) * inv, k3_bf_lo(v[1]) * inv,
                          k3_bf_hi(v[1]) * inv);
    o[1] = k3_pack_e4m3x4(k3_bf_lo(v[2]) * inv, k3_bf_hi(v[2]) * inv, k3_bf_lo(v[3]) * inv,
                          k3_bf_hi(v[3]) * inv);
    k3_st8_nt(y + i * 8, o);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const long long e = nv * 8 + threadIdx.x;
    y[e] = (uint8_t)(k3_pack_e4m3x2(k3_bf(x[e]) * inv, 0.0f) & 0xffu);
  }
}
