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
// Each thread owns 4 consecutive columns and 16 rows, loaded 4 rows at a time
// with the three taps carried in registers.  The logistic uses the hardware 2^x
// and reciprocal (as the reference's fast form does); the result is within one
// bf16 ulp of the CPU checker's exact logistic.
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
#define K9_CHUNK 4

K3_DEV void k9_unpack4(k3_u2 w, float* x) {
  x[0] = k3_bf_lo(w[0]); x[1] = k3_bf_hi(w[0]);
  x[2] = k3_bf_lo(w[1]); x[3] = k3_bf_hi(w[1]);
}
K3_DEV k3_u2 k9_ld4(const uint16_t* p) { return *(const k3_u2*)p; }

K3_DEV float k9_silu(float sb) { return sb * k3_sigmoid_fast(sb); }

K3_DEV k3_u2 k9_row(const float* t0, const float* t1, const float* t2, const float* x,
                    const float (*w)[4]) {
  float o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float y = t0[k] * w[0][k];
    y = __builtin_fmaf(t1[k], w[1][k], y);
    y = __builtin_fmaf(t2[k], w[2][k], y);
    y = __builtin_fmaf(x[k], w[3][k], y);
    o[k] = k9_silu(k3_land(y));
  }
  k3_u2 r;
  r[0] = k3_pack_bf2(o[0], o[1]);
  r[1] = k3_pack_bf2(o[2], o[3]);
  return r;
}

extern "C" __global__ void __launch_bounds__(128) kern_k3_span_gather(
    const uint16_t* __restrict__ partial, const float* __restrict__ cw, void* __restrict__ kda_base,
    const int* __restrict__ line_index, long long line_bytes, const float* __restrict__ wsm_partial,
    uint16_t* __restrict__ span_q, uint16_t* __restrict__ span_k, uint16_t* __restrict__ span_v,
    uint16_t* __restrict__ span_beta, uint16_t* __restrict__ span_flow,
    const int* __restrict__ span_at, int span) {
  const int at = span_at[0];
  const int row0 = blockIdx.z * K9_ROWS;
  if (row0 >= span) return;
  partial += (size_t)at * K9_KDA_FUSED;
  wsm_partial += (size_t)at * K9_WSM;

  if (blockIdx.y == 3) {
    // 8 threads per row: thread k lands beta for heads k, k + 8, ... and 16 flow columns
    const int i = row0 + (int)(threadIdx.x / 8), k = threadIdx.x % 8;
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
  const int c = (int)(blockIdx.x * 128 + threadIdx.x) * 4;
  uint16_t* __restrict__ out = s == 0 ? span_q : s == 1 ? span_k : span_v;
  uint16_t* win = (uint16_t*)((char*)kda_base + (long long)line_index[at] * line_bytes +
                              K9_REC_BYTES + (long long)s * K9_WIN_BYTES);
  float w[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 v = *(const float4*)(cw + (size_t)s * 4 * K9_INNER + (size_t)t * K9_INNER + c);
    w[t][0] = v.x; w[t][1] = v.y; w[t][2] = v.z; w[t][3] = v.w;
  }
  const uint16_t* __restrict__ col = partial + (size_t)s * K9_INNER + c;

  // x[j] = input row row0 - 3 + j
  float x[K9_CHUNK + 3][4];
  const bool first = blockIdx.z == 0;
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    if (first) k9_unpack4(k9_ld4(win + (size_t)t * K9_INNER + c), x[t]);
    else k9_unpack4(k9_ld4(col + (size_t)(row0 - 3 + t) * K9_KDA_FUSED), x[t]);
  }
  const int rend = min(row0 + K9_ROWS, span);
  for (int r0 = row0; r0 < rend; r0 += K9_CHUNK) {
    k3_u2 raw[K9_CHUNK];
#pragma unroll
    for (int r = 0; r < K9_CHUNK; ++r)
      if (r0 + r < rend) raw[r] = k9_ld4(col + (size_t)(r0 + r) * K9_KDA_FUSED);
#pragma unroll
    for (int r = 0; r < K9_CHUNK; ++r) {
      if (r0 + r < rend) {
        k9_unpack4(raw[r], x[3 + r]);
        *(k3_u2*)(out + (size_t)(r0 + r) * K9_INNER + c) = k9_row(x[r], x[r + 1], x[r + 2], x[r + 3], w);
      }
    }
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int k = 0; k < 4; ++k) x[t][k] = x[K9_CHUNK + t][k];
  }

  if (first) {
    // new window = x_{span-3 .. span-1}; all reads of the old window are done
    k3_u2 nt[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int i = span - 3 + t;
      nt[t] = i < 0 ? k9_ld4(win + (size_t)(i + 3) * K9_INNER + c)
                    : k9_ld4(col + (size_t)i * K9_KDA_FUSED);
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) *(k3_u2*)(win + (size_t)t * K9_INNER + c) = nt[t];
  }
}
