// Module k3_span_gather_v3+HEADS=24: KDA short conv + SiLU span gather (K9).
//
//   kern_k3_span_gather(partial, cw, kda_base, line_index, line_bytes, wsm_partial,
//                       span_q, span_k, span_v, span_beta, span_flow, span_at, span)
//       grid (INNER / 512, 4, ceil(span / 16))   block (128, 1, 1)
//
// Entry, parameters and geometry are the reference's (k3_span_gather_v3.cu:251;
// contract k3_span_gather_v2.cu:10-31; manifest op span_gather_v2,
// k3-tp4-prefill-16k.json:406197, line_bytes 1628160).  Batch rows
// [at, at + span), at = span_at[0], are consecutive tokens of one sequence.
//
// blockIdx.y = s < 3 (stream q, k, v), column c, span row i:
//   x_i   = f32(partial[at + i, s*INNER + c]) for i >= 0, win_s[i + 3][c] for i < 0
//   y_i   = x_{i-3} w0 + x_{i-2} w1 + x_{i-1} w2 + x_i w3,  w_t = cw[s][t][c] (f32),
//           evaluated as fma(x_i, w3, fma(x_{i-1}, w2, fma(x_{i-2}, w1, x_{i-3} w0)))
//   sb    = bf16(y_i);  out_s[i, c] = bf16(sb * sigmoid(sb))
// The window of stream s sits at kda_base + line_index[at] * line_bytes +
// HEADS*128*128*4 + s * 3*INNER*2 (k3_span_gather_v3.cu:286-287).  Only the
// z == 0 workgroup reads the old window (rows 0..2 need it) and, after those
// reads, writes the new one: win_s[t] = x_{span-3+t} (k3_span_gather.cu:31-35).
// blockIdx.y == 3: span_beta[h*span + i] = bf16(wsm[at+i, h]) for h < HEADS and
// span_flow[i, 0..128) = bf16(wsm[at+i, 96..224)) (k3_span_gather_v3.cu:267-281).
//
// Work split: a workgroup's tile is 512 columns x 16 rows of one stream; thread
// t owns 8 consecutive columns (one 16-byte vector per row) and one 8-row half
// of the tile (threads 0-63 rows 0-7, 64-127 rows 8-15).  All 11 rows a thread
// needs (its 8 rows and 3 taps) are loaded before any is used.  The second
// half's taps are the first half's last rows, so their re-read hits L2.  Only
// the first half of the z == 0 workgroup reads the old window, and it writes
// the new one after those reads.  beta / flow (y == 3) are landed once, by the
// x == 0 workgroups.  The logistic uses the hardware 2^x and reciprocal (as the
// reference's fast form does); the result is within one bf16 ulp of the CPU
// checker's exact logistic.
#include "../common/k3_dev.h"

#ifndef HEADS
#define HEADS 96
#endif
#define K9_INNER (HEADS * 128)
#define K9_KDA_FUSED (4 * K9_INNER)
#define K9_REC_BYTES ((long long)HEADS * 128 * 128 * 4)
#define K9_WIN_BYTES ((long long)3 * K9_INNER * 2)
#define K9_WSM 256
#define K9_WSM_FA 96
#define K9_ROWS 16

K3_DEV float k9_silu(float sb) { return sb * k3_sigmoid_fast(sb); }

// One output vector (8 columns) from taps t0..t2 and input x (raw bf16 words).
K3_DEV k3_u4 k9_row(k3_u4 t0, k3_u4 t1, k3_u4 t2, k3_u4 x, const float (*w)[8]) {
  k3_u4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = 2 * k + h;
      const float a0 = h ? k3_bf_hi(t0[k]) : k3_bf_lo(t0[k]);
      const float a1 = h ? k3_bf_hi(t1[k]) : k3_bf_lo(t1[k]);
      const float a2 = h ? k3_bf_hi(t2[k]) : k3_bf_lo(t2[k]);
      const float a3 = h ? k3_bf_hi(x[k]) : k3_bf_lo(x[k]);
      float y = a0 * w[0][e];
      y = __builtin_fmaf(a1, w[1][e], y);
      y = __builtin_fmaf(a2, w[2][e], y);
      y = __builtin_fmaf(a3, w[3][e], y);
      o[h] = k9_silu(k3_land(y));
    }
    r[k] = k3_pack_bf2(o[0], o[1]);
  }
  return r;
}

extern "C" __global__ void __launch_bounds__(128) kern_k3_span_gather(
    const uint16_t* __restrict__ partial, const float* __restrict__ cw, void* __restrict__ kda_base,
    const int* __restrict__ line_index, long long line_bytes, const float* __restrict__ wsm_partial,
    uint16_t* __restrict__ span_q, uint16_t* __restrict__ span_k, uint16_t* __restrict__ span_v,
    uint16_t* __restrict__ span_beta, uint16_t* __restrict__ span_flow,
    const int* __restrict__ span_at, int span) {
  const int at = span_at[0];
  const int tile0 = blockIdx.z * K9_ROWS;
  if (tile0 >= span) return;
  partial += (size_t)at * K9_KDA_FUSED;
  wsm_partial += (size_t)at * K9_WSM;

  if (blockIdx.y == 3) {
    if (blockIdx.x != 0) return;  // the six x workgroups would land identical values
    // 8 threads per row: thread k lands beta for heads k, k + 8, ... and 16 flow columns
    const int i = tile0 + (int)(threadIdx.x / 8), k = threadIdx.x % 8;
    if (i >= span) return;
    const float* row = wsm_partial + (size_t)i * K9_WSM;
    for (int h = k; h < HEADS; h += 8) span_beta[(size_t)h * span + i] = (uint16_t)k3_pack_bf2(row[h], 0.0f);
    const float4* fa = (const float4*)(row + K9_WSM_FA + k * 16);
    k3_u4 o0, o1;
    const float4 f0 = fa[0], f1 = fa[1], f2 = fa[2], f3 = fa[3];
    o0[0] = k3_pack_bf2(f0.x, f0.y); o0[1] = k3_pack_bf2(f0.z, f0.w);
    o0[2] = k3_pack_bf2(f1.x, f1.y); o0[3] = k3_pack_bf2(f1.z, f1.w);
    o1[0] = k3_pack_bf2(f2.x, f2.y); o1[1] = k3_pack_bf2(f2.z, f2.w);
    o1[2] = k3_pack_bf2(f3.x, f3.y); o1[3] = k3_pack_bf2(f3.z, f3.w);
    k3_st16(span_flow + (size_t)i * 128 + k * 16, o0);
    k3_st16(span_flow + (size_t)i * 128 + k * 16 + 8, o1);
    return;
  }

  const int s = blockIdx.y;
  const int half = threadIdx.x >> 6;
  const int c = (int)(blockIdx.x * 64 + (threadIdx.x & 63)) * 8;
  const int row0 = tile0 + half * 8;
  if (row0 >= span) return;
  const int nrow = min(8, span - row0);
  uint16_t* __restrict__ out = s == 0 ? span_q : s == 1 ? span_k : span_v;
  const uint16_t* __restrict__ col = partial + (size_t)s * K9_INNER + c;
  const bool first = blockIdx.z == 0 && half == 0;
  uint16_t* win = (uint16_t*)((char*)kda_base + (long long)line_index[at] * line_bytes +
                              K9_REC_BYTES + (long long)s * K9_WIN_BYTES);

  // x[j] = input row row0 - 3 + j (j < 3: taps), loaded before any use
  k3_u4 x[11];
#pragma unroll
  for (int t = 0; t < 3; ++t)
    x[t] = first ? k3_ld16(win + (size_t)t * K9_INNER + c)
                 : k3_ld16(col + (size_t)(row0 - 3 + t) * K9_KDA_FUSED);
#pragma unroll
  for (int r = 0; r < 8; ++r)
    x[3 + r] = k3_ld16_nt(col + (size_t)(row0 + min(r, nrow - 1)) * K9_KDA_FUSED);
  float w[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4* wp = (const float4*)(cw + (size_t)s * 4 * K9_INNER + (size_t)t * K9_INNER + c);
    const float4 a = wp[0], b = wp[1];
    w[t][0] = a.x; w[t][1] = a.y; w[t][2] = a.z; w[t][3] = a.w;
    w[t][4] = b.x; w[t][5] = b.y; w[t][6] = b.z; w[t][7] = b.w;
  }
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < nrow) k3_st16_nt(out + (size_t)(row0 + r) * K9_INNER + c, k9_row(x[r], x[r + 1], x[r + 2], x[r + 3], w));

  if (first) {
    // new window = x_{span-3 .. span-1}; this thread's old-window reads are done
    k3_u4 nt[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int i = span - 3 + t;
      // i < 0 (span < 3): old window row i + 3, still in x[0..2]
      nt[t] = i >= 0 ? k3_ld16(col + (size_t)i * K9_KDA_FUSED) : i == -3 ? x[0] : i == -2 ? x[1] : x[2];
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) k3_st16(win + (size_t)t * K9_INNER + c, nt[t]);
  }
}
