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
// Operator-shape probes (the byte patterns of three operators, with their
// arithmetic replaced by moves or xors):
//   k3h_probe_span_s<S>(src, d0, d1, d2, rows)   the KDA span gather: src
//       [rows, 4 * 3072] bf16 (bands 0-2 read), d_s [rows, 3072]; a workgroup of
//       128 S threads holds S tiles of 16 rows x 512 columns of one band, each
//       thread one 8-byte vector per row; the first tile of a workgroup also
//       loads the 3 rows before it (the conv taps), so S = 1 reads 3 rows in 16
//       twice and S = 2 (the typed call's shape) 3 in 32; S = 0: 16-row tiles of
//       128 threads without the tap rows (no re-read).  Grid 18 ceil(rows / 16
//       max(S, 1)).  Every input row vector is stored unchanged.
//   k3h_probe_gather(src, idx, dst, T, cols)   the weighted finalize: token t
//       = workgroup t (448 threads) gathers the rows src[idx[t, k]] with
//       idx >= 0 (k < 8) and writes their xor (zero if none) to dst[t]; each
//       thread 2 vectors of 16 bytes per row, every row load before any store.
//   k3h_probe_rowgather(src, idx, dst, R, cols)   the MXFP8 permute's payload:
//       dst[r] = src[idx[r]] (cols bytes, cols % 1024 == 0), one wave per row,
//       4 rows per 256-thread workgroup, all of a row's loads before its stores.
//   k3h_probe_rope(latent, k_rope, q, latent_out, q_out, T, H)   the MLA latent
//       norm + RoPE + q pack: one wave per token moves its latent and k_rope
//       rows and its H x 192 q values, as the operator's loads and stores do
//       (H must be 16; any other H stores nothing).
//   k3h_probe_push_t<NT>(src, snap, n0, n1, n2, n3, B)   the nb-0 residual push
//       at 4 ranks: one row read, five written (the snapshot slot and four
//       normed copies), grid B, NT = 128 (7 vectors per lane) or 896 (1).
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

// ---------------------------------------------------------------- operator shapes
template <int S>
K3_DEV void kp_span(const uint16_t* __restrict__ src, uint16_t* __restrict__ d0,
                    uint16_t* __restrict__ d1, uint16_t* __restrict__ d2, int rows) {
  constexpr int INNER = 3072, FUSED = 4 * INNER, XT = INNER / 512, SH = S > 0 ? S : 1;
  const int g = blockIdx.x / (3 * XT), sx = blockIdx.x % (3 * XT), st = sx / XT, x = sx % XT;
  const int half = threadIdx.x / 128, tid = threadIdx.x % 128;
  const int row0 = (g * SH + half) * 16;
  if (row0 >= rows) return;
  const int c = (x * 128 + tid) * 4;
  const uint16_t* col = src + (size_t)st * INNER + c;
  uint16_t* out = (st == 0 ? d0 : st == 1 ? d1 : d2) + c;
  k3_u2 v[19];
  const bool taps = S > 0 && half == 0;
#pragma unroll
  for (int t = 0; t < 3; ++t)
    if (taps) v[t] = __builtin_nontemporal_load((const k3_u2*)(col + (size_t)max(row0 - 3 + t, 0) * FUSED));
#pragma unroll
  for (int r = 0; r < 16; ++r)
    v[3 + r] = __builtin_nontemporal_load((const k3_u2*)(col + (size_t)min(row0 + r, rows - 1) * FUSED));
  k3_u2 tx = {0u, 0u};
  if (taps) tx = v[0] ^ v[1] ^ v[2];
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (row0 + r < rows) __builtin_nontemporal_store(v[3 + r] ^ (r == 0 ? tx : (k3_u2){0u, 0u}),
                                                     (k3_u2*)(out + (size_t)(row0 + r) * INNER));
}
extern "C" __global__ void __launch_bounds__(128) k3h_probe_span_s0(
    const uint16_t* src, uint16_t* d0, uint16_t* d1, uint16_t* d2, int rows) {
  kp_span<0>(src, d0, d1, d2, rows);
}
extern "C" __global__ void __launch_bounds__(128) k3h_probe_span_s1(
    const uint16_t* src, uint16_t* d0, uint16_t* d1, uint16_t* d2, int rows) {
  kp_span<1>(src, d0, d1, d2, rows);
}
extern "C" __global__ void __launch_bounds__(256) k3h_probe_span_s2(
    const uint16_t* src, uint16_t* d0, uint16_t* d1, uint16_t* d2, int rows) {
  kp_span<2>(src, d0, d1, d2, rows);
}

template <int NS>
K3_DEV void kp_gather_rows(const k3_u4* __restrict__ src, const int* srow, k3_u4* __restrict__ drow,
                           int nvec, int tid) {
  k3_u4 x[NS][2];
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      x[i][j] = __builtin_nontemporal_load(src + (size_t)srow[i] * nvec + min(tid + 448 * j, nvec - 1));
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    k3_u4 o = x[0][j];
#pragma unroll
    for (int i = 1; i < NS; ++i) o ^= x[i][j];
    __builtin_nontemporal_store(o, drow + min(tid + 448 * j, nvec - 1));
  }
}
extern "C" __global__ void __launch_bounds__(448) k3h_probe_gather(
    const k3_u4* __restrict__ src, const int* __restrict__ idx, k3_u4* __restrict__ dst, int T,
    int cols) {
  const int t = blockIdx.x, lane = threadIdx.x & 63, nvec = cols / 8;
  if (t >= T) return;
  const int p = lane < 8 ? idx[(size_t)t * 8 + lane] : -1;
  uint64_t m = __ballot(p >= 0);
  const int n = __builtin_popcountll(m);
  int srow[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    srow[i] = __builtin_amdgcn_readfirstlane(__shfl(p, m ? __builtin_ctzll(m) : 0, 64));
    m &= m - 1;
  }
  k3_u4* drow = dst + (size_t)t * nvec;
  switch (n) {
    case 0:
      for (int v = threadIdx.x; v < nvec; v += 448) __builtin_nontemporal_store((k3_u4){0u, 0u, 0u, 0u}, drow + v);
      break;
    case 1: kp_gather_rows<1>(src, srow, drow, nvec, threadIdx.x); break;
    case 2: kp_gather_rows<2>(src, srow, drow, nvec, threadIdx.x); break;
    case 3: kp_gather_rows<3>(src, srow, drow, nvec, threadIdx.x); break;
    case 4: kp_gather_rows<4>(src, srow, drow, nvec, threadIdx.x); break;
    case 5: kp_gather_rows<5>(src, srow, drow, nvec, threadIdx.x); break;
    case 6: kp_gather_rows<6>(src, srow, drow, nvec, threadIdx.x); break;
    case 7: kp_gather_rows<7>(src, srow, drow, nvec, threadIdx.x); break;
    default: kp_gather_rows<8>(src, srow, drow, nvec, threadIdx.x); break;
  }
}

extern "C" __global__ void __launch_bounds__(256) k3h_probe_rowgather(
    const k3_u4* __restrict__ src, const int* __restrict__ idx, k3_u4* __restrict__ dst, int R,
    int cols) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63, nvec = cols / 16;
  if (r >= R) return;
  const k3_u4* s = src + (size_t)idx[r] * nvec;
  k3_u4* d = dst + (size_t)r * nvec;
  for (int v0 = 0; v0 < nvec; v0 += 64 * 8) {
    k3_u4 x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = __builtin_nontemporal_load(s + min(v0 + lane + 64 * j, nvec - 1));
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (v0 + lane + 64 * j < nvec) __builtin_nontemporal_store(x[j], d + v0 + lane + 64 * j);
  }
}

// The nb-0 residual push at 4 ranks: row b of src (one 14,336-byte row) is
// stored to snap[8 b] (the snapshot slot's row stride) and to row B + b of each
// of n0..n3 (rank 1's rows of four normed_all buffers).  NT threads per row, each
// 7168 / (8 NT) vectors; every load first, then each vector to all five
// destinations.  NT = 128 is the operator's layout, NT = 896 one vector (one
// store per destination) per lane.
template <int NT>
K3_DEV void kp_push(const k3_u4* __restrict__ src, k3_u4* __restrict__ snap, k3_u4* __restrict__ n0,
                    k3_u4* __restrict__ n1, k3_u4* __restrict__ n2, k3_u4* __restrict__ n3, int B) {
  constexpr int RV = 7168 / 8, NV = RV / NT;
  const int b = blockIdx.x, t = threadIdx.x;
  if (b >= B) return;
  k3_u4 x[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) x[v] = __builtin_nontemporal_load(src + (size_t)b * RV + t + NT * v);
  const size_t o = (size_t)(B + b) * RV;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int u = t + NT * v;
    __builtin_nontemporal_store(x[v], snap + (size_t)b * 8 * RV + u);
    __builtin_nontemporal_store(x[v], n0 + o + u);
    __builtin_nontemporal_store(x[v], n1 + o + u);
    __builtin_nontemporal_store(x[v], n2 + o + u);
    __builtin_nontemporal_store(x[v], n3 + o + u);
  }
}
#define KP_PUSH(NT)                                                                            \
  extern "C" __global__ void __launch_bounds__(NT) k3h_probe_push_t##NT(                       \
      const k3_u4* src, k3_u4* snap, k3_u4* n0, k3_u4* n1, k3_u4* n2, k3_u4* n3, int B) {      \
    kp_push<NT>(src, snap, n0, n1, n2, n3, B);                                                 \
  }
KP_PUSH(128)
KP_PUSH(896)

// The MLA latent norm + RoPE + q pack: one wave per token (4 tokens per
// 256-thread workgroup) moves the token's latent row (1 KB, one vector per lane)
// and k_rope (128 B, lanes 0-7) to latent_out (1152 B) and its H x 192 q values
// (H * 24 vectors, in batches of 8 per lane) to q_out, every load of a token
// before its first store; the RoPE and the norm replaced by moves.
extern "C" __global__ void __launch_bounds__(256) k3h_probe_rope(
    const k3_u4* __restrict__ latent, const k3_u4* __restrict__ k_rope, const k3_u4* __restrict__ q,
    k3_u4* __restrict__ latent_out, k3_u4* __restrict__ q_out, int T, int H) {
  const int l = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T || H != 16) return;
  // H fixed at 16 (the config's heads): with a run-time count the compiler
  // guards each q load with a branch and a full wait, which serialises them
  constexpr int nvec = 16 * 24;
  const k3_u4 x = __builtin_nontemporal_load(latent + (size_t)t * 64 + l);
  k3_u4 kr = {0u, 0u, 0u, 0u};
  if (l < 8) kr = k_rope[(size_t)t * 8 + l];
  const k3_u4* qrow = q + (size_t)t * nvec;
  k3_u4* orow = q_out + (size_t)t * nvec;
  k3_u4 a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (64 * k < nvec) a[k] = __builtin_nontemporal_load(qrow + min(l + 64 * k, nvec - 1));
  __builtin_nontemporal_store(x, latent_out + (size_t)t * 72 + l);
  if (l < 8) __builtin_nontemporal_store(kr, latent_out + (size_t)t * 72 + 64 + l);
  for (int w0 = 0; w0 < nvec; w0 += 64 * 8) {
    if (w0 > 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (w0 + 64 * k < nvec) a[k] = __builtin_nontemporal_load(qrow + min(w0 + l + 64 * k, nvec - 1));
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (w0 + l + 64 * k < nvec) __builtin_nontemporal_store(a[k], orow + w0 + l + 64 * k);
  }
}

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
