// Module k3_moe_prefill_v{3,4}+...: the MoE prefill memory-bound family on gfx950.
//
//   kern_k3_moe_quant(x, q, sf, rows, cols)
//       grid (ceil(rows * cols / 32 / 256), 1, 1)   block (256, 1, 1)
//
// Entry names, parameter order and launch geometry are the reference module's
// (k3_moe_prefill_v4.cu:27-67; manifest ops moe_quant, moe_route_count,
// moe_route_tables, moe_route_scatter, moe_finalize).
#include "k3_mx.h"

// MXFP8 quantisation of a row-major bf16 tensor, 32-value blocks taken over the
// flat element order (k3_moe_prefill_v4.cu:111-140): sf[i] is the E8M0 scale
// of elements [32 i, 32 i + 32), q the e4m3 payload.
//
// The grid supplies one thread per block, as in the reference launch.  Inside a
// wave the 64 blocks of that wave are processed in four steps of 16 blocks:
// lane l takes 16 bytes at wave offset 1024 j + 16 l, so every load and store
// instruction covers one contiguous 1 KB (512 B for q) and the block amax is a
// quad max.
extern "C" __global__ void __launch_bounds__(256) kern_k3_moe_quant(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ sf,
    int rows, int cols) {
  const long long nblk = (long long)rows * cols / 32;
  const int l = threadIdx.x & 63;
  const long long first = (long long)blockIdx.x * blockDim.x + (threadIdx.x & ~63);
  k3_u4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long blk = first + 16 * j + (l >> 2);
    if (blk < nblk) v[j] = k3_ld16_nt(x + blk * 32 + (l & 3) * 8);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long blk = first + 16 * j + (l >> 2);
    if (blk < nblk) {  // uniform over the quad that shares the block
      k3_u2 qv;
      const int e = k3_mx_quad(v[j], &qv);
      k3_st8_nt(q + blk * 32 + (l & 3) * 8, qv);
      if ((l & 3) == 0) sf[blk] = (uint8_t)(e + 127);
    }
  }
}
