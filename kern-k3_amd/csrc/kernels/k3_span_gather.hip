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
// Work split: a tile is 512 columns x 16 rows of one stream; thread t of a
// tile owns 4 consecutive columns (one 8-byte vector per row) for all 16 rows,
// and all 19 row vectors (3 taps + 16 rows) and the weights are loaded (non-
// temporally) before any is used.  A workgroup of 128 * share threads holds
// `share` consecutive tiles of one column strip: under the manifest's block
// (128) one tile, under the typed call's (256) two, the second taking its three
// taps from the first tile's last input rows through LDS, so 3 rows in 32 are
// read twice instead of 3 in 16.  On MI355X this shape moves the span's bytes
// faster than 16-byte vectors over 8-row halves (6 tap rows per 16), than
// 16-byte vectors or 256-thread rows over 1024-column tiles, than four tiles
// per workgroup, than long column strips walked with the next block's loads in
// flight (the strips' row accesses drift apart in time and lose DRAM page
// locality: 120-146 us against 111 us at 16384 rows) and than any cacheable tap
// load (fast after a clean flush, 40% slower after a dirty one).  Only the
// z == 0 tile reads the old window, and it writes the new one after those
// reads.  beta / flow (y == 3) are landed once per row tile.  The logistic uses
// the hardware 2^x and reciprocal (as the reference's fast form does); the
// result is within one bf16 ulp of the CPU checker's exact logistic.
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
#define K9_XT (K9_INNER / 512)  // column tiles per stream (gridDim.x)

K3_DEV float k9_silu(float sb) { return sb * k3_sigmoid_fast(sb); }

K3_DEV void k9_unpack4(k3_u2 v, float* a) {
  a[0] = k3_bf_lo(v[0]); a[1] = k3_bf_hi(v[0]);
  a[2] = k3_bf_lo(v[1]); a[3] = k3_bf_hi(v[1]);
}

// One output vector (4 columns) from unpacked taps a0..a2 and input a3: conv fma
// chain, one bf16 landing per pair of values, SiLU, bf16 pack.
K3_DEV k3_u2 k9_row(const float* a0, const float* a1, const float* a2, const float* a3,
                    const float (*w)[4]) {
  k3_u2 r;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float y[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = 2 * k + h;
      float v = a0[e] * w[0][e];
      v = __builtin_fmaf(a1[e], w[1][e], v);
      v = __builtin_fmaf(a2[e], w[2][e], v);
      y[h] = __builtin_fmaf(a3[e], w[3][e], v);
    }
    const uint32_t sb = k3_pack_bf2(y[0], y[1]);
    r[k] = k3_pack_bf2(k9_silu(k3_bf_lo(sb)), k9_silu(k3_bf_hi(sb)));
  }
  return r;
}

K3_DEV k3_u2 k9_ld8_nt(const uint16_t* p) { return __builtin_nontemporal_load((const k3_u2*)p); }

#define K9_SHARE_MAX 4  // 16-row tiles per workgroup (block 128 x share)

extern "C" __global__ void __launch_bounds__(128 * K9_SHARE_MAX) kern_k3_span_gather(
    const uint16_t* __restrict__ partial, const float* __restrict__ cw, void* __restrict__ kda_base,
    const int* __restrict__ line_index, long long line_bytes, const float* __restrict__ wsm_partial,
    uint16_t* __restrict__ span_q, uint16_t* __restrict__ span_k, uint16_t* __restrict__ span_v,
    uint16_t* __restrict__ span_beta, uint16_t* __restrict__ span_flow,
    const int* __restrict__ span_at, int span) {
  // A workgroup of 128 * share threads (share = blockDim.x / 128: 1 under the
  // manifest's block, up to K9_SHARE_MAX) owns `share` consecutive 16-row tiles
  // of one column tile; thread group h (threads 128 h ..) owns tile h.  Tile h's
  // taps are tile h - 1's last three input rows, handed over through LDS, so the
  // workgroup reads the 3 rows before its first tile only.
  // Workgroups reach the XCDs round-robin by linear id.  The manifest launch has
  // 4 * K9_XT workgroups per row tile but only 3 * K9_XT + 1 with work, so the
  // tiles are renumbered: linear ids [0, 3 K9_XT ng) are the stream tile groups
  // (column tile fastest, then stream, then row group), the next ng ids the
  // beta / flow groups, and the rest exit.  Every XCD then gets the same share.
  const int share = (int)blockDim.x / 128, half = (int)threadIdx.x / 128;
  const int tid = (int)threadIdx.x % 128;
  const uint32_t nz = (uint32_t)(span + K9_ROWS - 1) / K9_ROWS;
  const uint32_t ng = (nz + share - 1) / share;
  const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  uint32_t bx, by, bg;
  if (L < 3 * K9_XT * ng) {
    bg = L / (3 * K9_XT);
    by = L % (3 * K9_XT) / K9_XT;
    bx = L % K9_XT;
  } else if (L < (3 * K9_XT + 1) * ng) {
    bg = L - 3 * K9_XT * ng;
    by = 3;
    bx = 0;
  } else {
    return;
  }
  const uint32_t bz = bg * share + half;
  const int at = span_at[0];
  const int tile0 = bz * K9_ROWS;
  partial += (size_t)at * K9_KDA_FUSED;
  wsm_partial += (size_t)at * K9_WSM;

  if (by == 3) {
    // 8 threads per row: thread k lands beta for heads k, k + 8, ... and 16 flow columns
    const int i = tile0 + tid / 8, k = tid % 8;
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

  const int s = by;
  const int c = (int)(bx * 128 + tid) * 4;
  const int row0 = tile0;
  // rows of this tile; 0 for a thread group past the span's last tile (it loads
  // and stores nothing but still meets the workgroup barrier)
  const int nrow = max(0, min(K9_ROWS, span - row0));
  uint16_t* __restrict__ out = s == 0 ? span_q : s == 1 ? span_k : span_v;
  const uint16_t* __restrict__ col = partial + (size_t)s * K9_INNER + c;
  const bool first = bz == 0;
  uint16_t* win = (uint16_t*)((char*)kda_base + (long long)line_index[at] * line_bytes +
                              K9_REC_BYTES + (long long)s * K9_WIN_BYTES);

  // Loads in first-use order (weights, taps, rows), all issued before any use.
  float w[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const k3_u4 a = k3_ld16(cw + (size_t)s * 4 * K9_INNER + (size_t)t * K9_INNER + c);
#pragma unroll
    for (int k = 0; k < 4; ++k) w[t][k] = __uint_as_float(a[k]);
  }
  // x[j] = input row row0 - 3 + j (j < 3: taps)
  k3_u2 x[K9_ROWS + 3];
  if (half == 0) {
#pragma unroll
    for (int t = 0; t < 3; ++t)
      x[t] = first ? *(const k3_u2*)(win + (size_t)t * K9_INNER + c)
                   : k9_ld8_nt(col + (size_t)(row0 - 3 + t) * K9_KDA_FUSED);
  }
  if (nrow > 0) {
#pragma unroll
    for (int r = 0; r < K9_ROWS; ++r)
      x[3 + r] = k9_ld8_nt(col + (size_t)(row0 + min(r, nrow - 1)) * K9_KDA_FUSED);
  }
  if (share > 1) {
    __shared__ k3_u2 taps_s[K9_SHARE_MAX - 1][3][128];
    if (half < share - 1 && nrow > 0) {
#pragma unroll
      for (int t = 0; t < 3; ++t) taps_s[half][t][tid] = x[K9_ROWS + t];
    }
    __syncthreads();
    if (half > 0) {
#pragma unroll
      for (int t = 0; t < 3; ++t) x[t] = taps_s[half - 1][t][tid];
    }
  }
  if (nrow == 0) return;

  // slide over the rows: each input row is unpacked once
  float a[4][4];
  k9_unpack4(x[0], a[0]);
  k9_unpack4(x[1], a[1]);
  k9_unpack4(x[2], a[2]);
#pragma unroll
  for (int r = 0; r < K9_ROWS; ++r) {
    k9_unpack4(x[3 + r], a[(r + 3) & 3]);
    const k3_u2 o = k9_row(a[r & 3], a[(r + 1) & 3], a[(r + 2) & 3], a[(r + 3) & 3], w);
    if (r < nrow) __builtin_nontemporal_store(o, (k3_u2*)(out + (size_t)(row0 + r) * K9_INNER + c));
  }

  if (first) {
    // new window = x_{span-3 .. span-1}; this thread's old-window reads are done
    k3_u2 nt[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int i = span - 3 + t;
      // i < 0 (span < 3): old window row i + 3, still in x[0..2]
      nt[t] = i >= 0 ? *(const k3_u2*)(col + (size_t)i * K9_KDA_FUSED) : i == -3 ? x[0] : i == -2 ? x[1] : x[2];
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) *(k3_u2*)(win + (size_t)t * K9_INNER + c) = nt[t];
  }
}
