// Module k3h_mla_rope: MLA latent RMSNorm + interleaved RoPE + q packing.
// No reference entry: the reference lands the rope columns as a plain bf16 copy
// (k3_mla_prep_v2.cu:205-210) and carries the rope dims into K through identity
// rows of the kv_b augmentation (k3_weight_prep.cu:81-93).
//
//   k3h_mla_rope_pack(latent, k_rope, q, gamma_kv, positions, latent_out, q_out,
//                     theta, eps, T, H)
//       grid ceil(T / 4), block 256: one wave per token
//
// Per token t at position p = positions[t]:
//   latent_out[t, 0..512)   = bf16(bf16(latent * r) (x) gamma_kv),
//                             r = 1 / sqrt(sum(latent^2) / 512 + eps)
//   latent_out[t, 512..576) = rope(k_rope[t])
//   q_out[t, h, 0..128)     = q[t, h, 0..128)              (nope dims, copied)
//   q_out[t, h, 128..192)   = rope(q[t, h, 128..192))
// rope: pairs (x[2j], x[2j+1]), j < 32, rotated by a_j = p * theta^(-2j/64):
//   y0 = x0 cos a_j - x1 sin a_j,  y1 = x0 sin a_j + x1 cos a_j,  one bf16 landing,
// evaluated as y0 = fma(x0, c, -(x1 s)), y1 = fma(x0, s, x1 c) with c, s the f32
// roundings of cos / sin computed in double (lanes 0..31 of the wave, one pair
// each, shared through LDS).  The sum of squares is 8 serial fmas per lane and a
// 64-lane xor butterfly (32, 16, ..., 1).  A wave's loads (latent, k_rope and
// the first 8 q vectors per lane) are issued before the fp64 angles and the
// barrier, so that their latency covers the angle computation.  q is [T, H, 192] contiguous, the
// latent row [T, 576] (16-byte aligned rows).
#include "../common/k3_dev.h"

#define K3_KV 512
#define K3_ROPE 64
#define K3_LAT (K3_KV + K3_ROPE)
#define K3_QH 192

K3_DEV void k3_rot2(float x0, float x1, float c, float s, float* y0, float* y1) {
  *y0 = __builtin_fmaf(x0, c, -(x1 * s));
  *y1 = __builtin_fmaf(x0, s, x1 * c);
}

// Rotate the four pairs of one 16-byte vector (8 bf16) starting at pair j0.
K3_DEV k3_u4 k3_rope_vec(k3_u4 v, const float2* cs, int j0) {
  k3_u4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float2 t = cs[j0 + k];
    float y0, y1;
    k3_rot2(k3_bf_lo(v[k]), k3_bf_hi(v[k]), t.x, t.y, &y0, &y1);
    o[k] = k3_pack_bf2(y0, y1);
  }
  return o;
}

extern "C" __global__ void __launch_bounds__(256) k3h_mla_rope_pack(
    const uint16_t* __restrict__ latent, const uint16_t* __restrict__ k_rope,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ gamma_kv,
    const long long* __restrict__ positions, uint16_t* __restrict__ latent_out,
    uint16_t* __restrict__ q_out, float theta, float eps, int T, int H) {
  __shared__ float2 s_cs[4][K3_ROPE / 2];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wv;
  const bool live = t < T;
  const int tt = live ? t : T - 1;  // loads stay in bounds; stores are predicated

  // every load of the first batch goes out before the angles (fp64) and the
  // barrier: the latent row, k_rope (8 lanes) and up to 8 q vectors per lane
  const int nvec = H * (K3_QH / 8);  // q: H heads x 24 vectors; 16..23 are rope dims
  const uint16_t* qrow = q + (size_t)tt * H * K3_QH;
  const k3_u4 x = k3_ld16_nt(latent + (size_t)tt * K3_KV + 8 * l);
  k3_u4 kr = {0u, 0u, 0u, 0u};
  if (l < K3_ROPE / 8) kr = k3_ld16(k_rope + (size_t)tt * K3_ROPE + 8 * l);
  k3_u4 a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (64 * k < nvec) a[k] = k3_ld16_nt(qrow + 8 * min(l + 64 * k, nvec - 1));
  if (l < K3_ROPE / 2) {
    const double inv = pow((double)theta, -(double)(2 * l) / (double)K3_ROPE);
    const double ang = (double)positions[tt] * inv;
    s_cs[wv][l] = make_float2((float)cos(ang), (float)sin(ang));
  }
  // latent RMSNorm: lane l owns elements 8l .. 8l + 7
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a0 = k3_bf_lo(x[k]), b0 = k3_bf_hi(x[k]);
    sq = __builtin_fmaf(a0, a0, sq);
    sq = __builtin_fmaf(b0, b0, sq);
  }
  sq += __shfl_xor(sq, 32, 64);
  sq = k3_sum32(sq);
  const float r = k3_rsqrt_cr(__builtin_fmaf(sq, 1.0f / K3_KV, eps));
  __syncthreads();  // s_cs ready
  const float2* cs = s_cs[wv];
  if (!live) return;

  const k3_u4 g = k3_ld16(gamma_kv + 8 * l);
  k3_u4 nv;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    nv[k] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(x[k]) * r, k3_bf_hi(x[k]) * r), g[k]);
  uint16_t* lrow = latent_out + (size_t)t * K3_LAT;
  k3_st16_nt(lrow + 8 * l, nv);
  if (l < K3_ROPE / 8) k3_st16_nt(lrow + K3_KV + 8 * l, k3_rope_vec(kr, cs, 4 * l));
  uint16_t* orow = q_out + (size_t)t * H * K3_QH;
  // batches of 8 vectors per lane, all loaded before the first store (indices
  // past the row are clamped for the load and skipped for the store); the first
  // batch was loaded above
  for (int w0 = 0; w0 < nvec; w0 += 64 * 8) {
    if (w0 > 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (w0 + 64 * k < nvec) a[k] = k3_ld16_nt(qrow + 8 * min(w0 + l + 64 * k, nvec - 1));
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int w = w0 + l + 64 * k;
      const int v = w % (K3_QH / 8);
      if (w < nvec) k3_st16_nt(orow + 8 * w, v < 16 ? a[k] : k3_rope_vec(a[k], cs, 4 * (v - 16)));
    }
  }
}
