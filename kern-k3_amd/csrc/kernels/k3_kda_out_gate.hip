// Module k3_kda_out_gate_v3+HEADS=24[+K11_RMS_EPS=1e-6f]: the KDA output gate (K11).
//
//   kern_k3_kda_out_gate(attn, gate_partial, gamma_o, gated, span_at, span)
//       grid (span, HEADS / 8, 1)   block (128, 1, 1)
//
// Entry, parameters and geometry are the reference's (k3_kda_out_gate_v3.cu:36;
// contract k3_kda_out_gate_v2.cu:5-23; manifest op kda_out_gate_v2,
// k3-tp4-prefill-16k.json:406169).  For span row i, head h, dv < 128, b = at + i:
//   a  = f32(attn[i, h*128 + dv]);   r = rsqrt(sum_dv a^2 / 128 + eps)
//   o  = bf16(a * r * gamma_o[dv]);  gt = bf16(sigmoid(g)), g = gate_partial[b, 3*INNER + h*128 + dv]
//   gated[b, h*128 + dv] = bf16(f32(o) * f32(gt))
// Thread layout of the reference: 8 heads per workgroup, 16 lanes per head, 8
// consecutive elements (one 16-byte vector) per lane; the sum of squares is 8
// serial fmas per lane and a 16-lane xor butterfly (8, 4, 2, 1), which on a
// 64-lane wave is four heads per wave with the butterfly inside 16-lane rows.
// r is 1 / sqrt, correctly rounded (the CPU checker matches it exactly); the
// logistic uses the hardware 2^x and reciprocal (about 1 f32 ulp each), so
// gated is within one bf16 ulp of the checker's exact logistic.
#include "../common/k3_dev.h"

#ifndef HEADS
#define HEADS 96
#endif
#define K11_INNER (HEADS * 128)
#define K11_KDA_FUSED (4 * K11_INNER)
// The norm's eps is a compile-time define, as in the reference
// (k3_kda_out_gate_v3.cu:25): 1e-5 by default, 1e-6 in the +K11_RMS_EPS=1e-6f build.
#ifndef K11_RMS_EPS
#define K11_RMS_EPS 1e-5f
#endif
static_assert(HEADS % 8 == 0, "HEADS must be a multiple of 8");

// One (row, 16-byte column vector) of the gate: the per-head sum of squares
// runs over the 16 lanes of the head (a 16-lane row of the wave).
K3_DEV k3_u4 k11_gate_vec(k3_u4 av, k3_u4 gv, const float* gm) {
  float a[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) { a[2 * k] = k3_bf_lo(av[k]); a[2 * k + 1] = k3_bf_hi(av[k]); }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(a[k], a[k], ss);
  ss = k3_sum16(ss);
  const float r = k3_rsqrt_cr(__builtin_fmaf(ss, 1.0f / 128.0f, K11_RMS_EPS));
  k3_u4 out;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float o0 = k3_land(a[2 * k] * r * gm[2 * k]);
    const float o1 = k3_land(a[2 * k + 1] * r * gm[2 * k + 1]);
    const float t0 = k3_land(k3_sigmoid_fast(k3_bf_lo(gv[k])));
    const float t1 = k3_land(k3_sigmoid_fast(k3_bf_hi(gv[k])));
    out[k] = k3_pack_bf2(o0 * t0, o1 * t1);
  }
  return out;
}

// Tiles are taken in memory order: linear workgroup id L (x fastest) is span row
// L / gridDim.y, column block L % gridDim.y, so neighbouring workgroups read
// neighbouring 1 KB pieces of one row instead of one piece from each of
// consecutive rows.  Same grid, same tiles, same per-element work.
extern "C" __global__ void __launch_bounds__(128) kern_k3_kda_out_gate(
    const uint16_t* __restrict__ attn, const uint16_t* __restrict__ gate_partial,
    const float* __restrict__ gamma_o, uint16_t* __restrict__ gated,
    const int* __restrict__ span_at, int span) {
  const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y;
  const int i = (int)(L / gridDim.y);
  if (i >= span) return;
  const int h = (int)(L % gridDim.y) * 8 + threadIdx.x / 16;
  const int d0 = (threadIdx.x % 16) * 8;
  const size_t col = (size_t)h * 128 + d0;
  const int b = span_at[0] + i;

  const k3_u4 av = k3_ld16_nt(attn + (size_t)i * K11_INNER + col);
  const k3_u4 gv = k3_ld16_nt(gate_partial + (size_t)b * K11_KDA_FUSED + 3 * K11_INNER + col);
  const float4 gm0 = *(const float4*)(gamma_o + d0);
  const float4 gm1 = *(const float4*)(gamma_o + d0 + 4);
  const float gm[8] = {gm0.x, gm0.y, gm0.z, gm0.w, gm1.x, gm1.y, gm1.z, gm1.w};
  k3_st16_nt(gated + (size_t)b * K11_INNER + col, k11_gate_vec(av, gv, gm));
}
