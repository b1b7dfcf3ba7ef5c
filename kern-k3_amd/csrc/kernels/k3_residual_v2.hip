// Module k3_residual_v2[+LAND_BF16=1][+K3_EPS=...]: the K1 residual family.
//
//   kern_k3_attnres_rms(prefix, blocks, sw, gamma, normed, nb, snapshot, B)
//   kern_k3_land_add_attnres_rms(partial, prefix, blocks, sw, gamma,
//                                prefix2, normed, nb, snapshot, B)
//   kern_k3_land_add2(p1, p2, prefix2, hidden, two, B)
//
// Entry names, parameter order and launch geometry are the reference module's
// (k3_residual_v2.cu:260, 295, 349; manifest ops attnres_rms_v2,
// land_add_attnres_rms_bf16_v2, land_add2_v2): grid (B, 1, 1), block (128, 1, 1),
// no dynamic LDS.  A block index b >= B returns at once.  The row body is in
// k3_residual_row.h.
#include "k3_residual_row.h"

// K1a: mixing + RMS of the prefix row; with `snapshot` and nb < 8 the prefix row
// is first copied to blocks[b, nb] (k3_residual_v2.cu:260-284).
extern "C" __global__ void __launch_bounds__(K3_RES_THREADS) kern_k3_attnres_rms(
    const uint16_t* __restrict__ prefix, uint16_t* __restrict__ blocks,
    const float* __restrict__ sw, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ normed, int nb, int snapshot, int B) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const int t = threadIdx.x;
  if (nb < 0 || nb > K3_NB_MAX) return;
  k3_u4 pv[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_ld16_nt(prefix + (size_t)b * K3_H + k3_vec_off(t, v));
  if (snapshot && nb < K3_NB_MAX) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v)
      k3_st16_nt(blocks + ((size_t)b * K3_NB_MAX + nb) * K3_H + k3_vec_off(t, v), pv[v]);
  }
  k3_attnres_rms_row<-1>(blocks + (size_t)b * K3_NB_MAX * K3_H, pv, sw, gamma,
                         normed + (size_t)b * K3_H, nb, K3_EPS, t);
}

// K1b: landing add, then K1a's row body on the new prefix (k3_residual_v2.cu:295-345).
extern "C" __global__ void __launch_bounds__(K3_RES_THREADS) kern_k3_land_add_attnres_rms(
    const k3_land_t* __restrict__ partial, const uint16_t* __restrict__ prefix,
    const uint16_t* __restrict__ blocks, const float* __restrict__ sw,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ prefix2,
    uint16_t* __restrict__ normed, int nb, int snapshot, int B) {
  if (nb < 0 || nb > K3_NB_MAX) return;
  k3_land_add_attnres_rms_body<-1>(partial, prefix, blocks, sw, gamma, prefix2, normed, nb,
                                   snapshot, B);
}

// K1c: hidden = bf16(f32(prefix2) + f32(bf16(p1)) [+ f32(bf16(p2))]), p1/p2 f32
// (k3_residual_v2.cu:349-392).  The sum is left to right, one final rounding.
extern "C" __global__ void __launch_bounds__(K3_RES_THREADS) kern_k3_land_add2(
    const float* __restrict__ p1, const float* __restrict__ p2,
    const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden, int two, int B) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    const size_t off = (size_t)b * K3_H + k3_vec_off(t, v);
    const float4 a1 = k3_ld16f_nt(p1 + off);
    const float4 b1 = k3_ld16f_nt(p1 + off + 4);
    const float f1[8] = {a1.x, a1.y, a1.z, a1.w, b1.x, b1.y, b1.z, b1.w};
    float f2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (two) {
      const float4 a2 = k3_ld16f_nt(p2 + off);
      const float4 b2 = k3_ld16f_nt(p2 + off + 4);
      f2[0] = a2.x; f2[1] = a2.y; f2[2] = a2.z; f2[3] = a2.w;
      f2[4] = b2.x; f2[5] = b2.y; f2[6] = b2.z; f2[7] = b2.w;
    }
    const k3_u4 pr = k3_ld16_nt(prefix2 + off);
    k3_u4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x = k3_bf_lo(pr[j]) + k3_land(f1[2 * j]);
      float y = k3_bf_hi(pr[j]) + k3_land(f1[2 * j + 1]);
      if (two) {
        x += k3_land(f2[2 * j]);
        y += k3_land(f2[2 * j + 1]);
      }
      o[j] = k3_pack_bf2(x, y);
    }
    k3_st16_nt(hidden + off, o);
  }
}
