// Module k3h_fused: operators with no single reference entry.
//
//   k3h_residual_rms_mxfp8(x, residual, gamma, residual_out, q, sf, normed, eps, B)
//       grid (ceil(B / 2), 1, 1)   block (256, 1, 1)
//
// Residual add + RMSNorm + MXFP8: the K1b landing with nb = 0 and snapshot = 0
// (k3_residual_v2.cu:295-345 with the row body of 107-257 reduced to its RMS
// part), whose normed row is quantised by the kern_k3_moe_quant block rule
// (k3_moe_prefill_v4.cu:111-140) without ever being stored as bf16:
//   residual_out = bf16(f32(residual) + f32(x))
//   normed       = bf16(bf16(residual_out * r) (x) gamma),
//                  r = 1 / sqrt(sum(residual_out^2) / 7168 + eps)
//   sf[b, k]     = e_k + 127, q[b, 32k + i] = e4m3(normed[32k + i] * 2^-e_k)
// `normed` may be null; when given, the bf16 normed row is stored as well (the
// test path uses it to check q/sf against the exact normed values).
//
// HBM traffic per row: 2 x 14336 B read, 14336 + 7168 + 224 B written (gamma
// is 14 KB shared by all rows and stays in L2).  A 256-thread workgroup holds
// two rows, one per 128-thread half; within a half, thread t owns the 16-byte
// vectors t + 128 v of its row (the K1 ownership, so the sum of squares has the
// K1 order), and a 32-value MX block is the vectors of four consecutive lanes
// at the same v.  Measured back to back at 16384 rows: one, two and four rows
// per workgroup 134.8, 134.5 and 137.4 us.  The E8M0 bytes of four quads are
// gathered into one lane and stored as a word, after the quantisation loop.  A half whose row is past B
// still takes part in the workgroup barrier but stores nothing.
//
// Wait discipline: the vector memory counter counts stores as well as loads,
// in issue order, so waiting for a load also waits for every store issued
// before it.  gamma is therefore loaded one vector ahead of its use (the load
// for v + 1 goes out before the stores of v), and the quantisation loop has no
// branch (normed is a template parameter, the E8M0 words leave after the
// loop), which lets the compiler wait for exactly the load it needs.
#include "k3_residual_row.h"
#include "k3_mx.h"

#define K3_FUSED_ROWS 2

template <bool NORMED>
K3_DEV void k3h_fused_rows(const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
                           const uint16_t* __restrict__ gamma, uint16_t* __restrict__ residual_out,
                           uint8_t* __restrict__ q, uint8_t* __restrict__ sf, uint16_t* __restrict__ normed,
                           float eps, int B) {
  __shared__ float s_red[K3_FUSED_ROWS * K3_NHW];
  const int half = threadIdx.x / K3_RES_THREADS;
  const int t = threadIdx.x % K3_RES_THREADS;
  const int b = blockIdx.x * K3_FUSED_ROWS + half;
  const bool live = b < B;
  const size_t row = (size_t)(live ? b : 0) * K3_H;

  // Loads are unconditional (a dead half reads row 0, which exists because the
  // grid only covers B >= 1): a predicated load would be compiled as a branch
  // with a full wait per vector and lose the memory-level parallelism.
  k3_u4 rv[K3_KVPT], xv[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    const size_t off = row + k3_vec_off(t, v);
    rv[v] = k3_ld16_nt(residual + off);
    xv[v] = k3_ld16_nt(x + off);
  }
  k3_u4 gnext = k3_ld16(gamma + k3_vec_off(t, 0));
  // every load of the row is issued before any arithmetic uses one (without the
  // fence the scheduler interleaves the first sums and waits with the later
  // loads, and fewer loads are in flight)
  __builtin_amdgcn_sched_barrier(0);
  k3_u4 pv[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_add_land(rv[v], xv[v]);

  const float tot = k3_block_sum128(k3_row_sumsq(pv), s_red + half * K3_NHW, t);
  if (!live) return;  // no barrier follows
  // residual_out leaves after the reduction, beside the payload (0.8% faster
  // than storing it before the barrier)
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt(residual_out + row + k3_vec_off(t, v), pv[v]);
  const float r = k3_row_rscale(tot, eps);
  uint32_t sfw[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    const int u = k3_vec_off(t, v);
    const k3_u4 g = gnext;
    if (v + 1 < K3_KVPT) gnext = k3_ld16(gamma + k3_vec_off(t, v + 1));
    k3_u4 nv;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      nv[j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(pv[v][j]) * r, k3_bf_hi(pv[v][j]) * r), g[j]);
    k3_u2 qv;
    const uint32_t sfb = (uint32_t)(k3_mx_quad(nv, &qv) + 127);
    k3_st8_nt(q + row + u, qv);
    // lane 16m gathers the bytes of quads 4m .. 4m + 3 (lanes 16m + 4k)
    sfw[v] = sfb | (k3_swz_xor_u32<4>(sfb) << 8) | (k3_swz_xor_u32<8>(sfb) << 16) |
             (k3_swz_xor_u32<12>(sfb) << 24);
    if (NORMED) k3_st16(normed + row + u, nv);
  }
  if ((t & 15) == 0) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v)
      *(uint32_t*)(sf + (size_t)b * (K3_H / 32) + (k3_vec_off(t, v) >> 5)) = sfw[v];
  }
}

extern "C" __global__ void __launch_bounds__(K3_RES_THREADS * K3_FUSED_ROWS) k3h_residual_rms_mxfp8(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ residual_out,
    uint8_t* __restrict__ q, uint8_t* __restrict__ sf, uint16_t* __restrict__ normed,
    float eps, int B) {
  if (normed) k3h_fused_rows<true>(x, residual, gamma, residual_out, q, sf, normed, eps, B);
  else k3h_fused_rows<false>(x, residual, gamma, residual_out, q, sf, normed, eps, B);
}

// Plain 16-byte streaming copy (measurement support: the HBM ceiling and the
// byte-counter calibration).  grid ceil(n16 / 256), block 256.
extern "C" __global__ void __launch_bounds__(256) k3h_stream_copy(
    const k3_u4* __restrict__ src, k3_u4* __restrict__ dst, long long n16) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}
