// Modules k3_residual_push, k3_residual_push_v3, k3_residual_push_stats and
// k3_residual_push_add2: res_in, the attention residual + RMSNorm whose normed
// row is stored into every TP rank's `normed_all` (the all-gather folded into
// the producer).  One entry per module, `kern_k3_attnres_rms_push`, with the
// module's parameter list:
//
//   push, push_v3 (K3_PUSH = 1; k3_residual_push.cu:320, k3_residual_push_v3.cu:324):
//     (prefix, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks)
//   push_stats (K3_PUSH = 2; k3_residual_push_stats.cu:354):
//     (prefix, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks,
//      sw_mlp, stats)
//   push_add2 (K3_PUSH = 3; k3_residual_push_add2.cu:362; manifest op attnres_rms_push_add2):
//     (blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks,
//      sw_mlp, stats, p1, p2, prefix2, hidden, two)
//
// grid (B, 1, 1), block (128, 1, 1) (manifest ceil_div(tokens, 4) rows per rank).
//
// Typed-call entries k3h_attnres_rms_push_nb{K}s (K = 1..8, nb == K; same
// parameter list as the module's entry, block 256): the vector-split row body
// (k3_residual_split.h), every candidate held on chip from pass 1 to pass 2,
// the same bits; and k3h_attnres_rms_push_nb0w896 (nb == 0, block 896: one
// vector of the row per lane, below), the same bits as the nb-0 branch.
//
// Row b of this rank lands at row rank * B + b of every rank's normed_all: the
// local copy through `normed_all`, the others through dst_peer[q] (q < nranks,
// q != rank; nranks is capped at 8), each a device address of rank q's
// normed_all (an xGMI peer mapping on a multi-GPU node).  The arithmetic is the
// K1a row body (kern_k3_attnres_rms); push_stats also writes the candidates'
// (sum x^2, sum x * sw_mlp) to stats[b] for res_mlp, and push_add2 first forms
// the row as hidden = bf16(f32(prefix2) + f32(p1) [+ f32(p2)]) (bf16 inputs,
// left to right, one rounding; kern_k3_land_add2_bf16), stores it to `hidden`
// and uses it as the prefix candidate.  With snapshot and nb < 8 the prefix row
// is copied to blocks[b, nb] first.  No fence: the stores are released by the
// arrival barrier, a later launch on the same stream.
#include "k3_residual_row.h"
#include "k3_residual_split.h"

#ifndef K3_PUSH
#define K3_PUSH 1
#endif

#define K3_PUSH_EPS 1e-5f

#if K3_PUSH == 3
// hidden = bf16(f32(prefix2) + f32(p1) [+ f32(p2)]) for this thread's vectors,
// left to right, one rounding
K3_DEV k3_u4 k3_add2_vec(k3_u4 pv, k3_u4 a, k3_u4 e, int two) {
  k3_u4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x = k3_bf_lo(pv[j]) + k3_bf_lo(a[j]);
    float y = k3_bf_hi(pv[j]) + k3_bf_hi(a[j]);
    if (two) {
      x += k3_bf_lo(e[j]);
      y += k3_bf_hi(e[j]);
    }
    o[j] = k3_pack_bf2(x, y);
  }
  return o;
}

K3_DEV void k3_push_land_add2(const uint16_t* __restrict__ p1, const uint16_t* __restrict__ p2,
                              const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden,
                              int two, size_t row, int t, k3_u4* pv) {
  // all loads first, then the adds and the hidden stores
  k3_u4 a[K3_KVPT], e[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    a[v] = k3_ld16_nt(p1 + row + k3_vec_off(t, v));
    pv[v] = k3_ld16_nt(prefix2 + row + k3_vec_off(t, v));
  }
  if (two) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) e[v] = k3_ld16_nt(p2 + row + k3_vec_off(t, v));
  }
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_add2_vec(pv[v], a[v], e[v], two);
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) k3_st16(hidden + row + k3_vec_off(t, v), pv[v]);
}
#endif

extern "C" __global__ void __launch_bounds__(K3_RES_THREADS) kern_k3_attnres_rms_push(
#if K3_PUSH != 3
    const uint16_t* __restrict__ prefix,
#endif
    uint16_t* __restrict__ blocks, const float* __restrict__ sw,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ normed_all,
    const unsigned long long* __restrict__ dst_peer, int nb, int snapshot, int B, int rank,
    int nranks
#if K3_PUSH >= 2
    , const float* __restrict__ sw_mlp, float* __restrict__ stats
#endif
#if K3_PUSH == 3
    , const uint16_t* __restrict__ p1, const uint16_t* __restrict__ p2,
    const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden, int two
#endif
) {
  const int b = blockIdx.x;
  if (b >= B) return;
  if (nb < 0 || nb > K3_NB_MAX) return;
  const int t = threadIdx.x;
  const int nr = nranks < K3_MAX_RANKS ? nranks : K3_MAX_RANKS;
  const long long dst_off = ((long long)rank * B + b) * K3_H;
  const size_t row = (size_t)b * K3_H;

  if (nb == 0) {
    // the first layer's res_in (the mix is the identity): every load of the row
    // first (the prefix or its land_add2 operands, gamma), the reduction, then
    // the stores (hidden, the snapshot slot, the normed copies), so that no load
    // waits behind a store; the arithmetic of the general body at nb == 0
    __shared__ float s_red0[K3_NHW];
    k3_u4 pv[K3_KVPT], g[K3_KVPT];
#if K3_PUSH == 3
    k3_u4 a[K3_KVPT], e[K3_KVPT];
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) {
      a[v] = k3_ld16_nt(p1 + row + k3_vec_off(t, v));
      pv[v] = k3_ld16_nt(prefix2 + row + k3_vec_off(t, v));
    }
    if (two) {
#pragma unroll
      for (int v = 0; v < K3_KVPT; ++v) e[v] = k3_ld16_nt(p2 + row + k3_vec_off(t, v));
    }
#else
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_ld16_nt(prefix + row + k3_vec_off(t, v));
#endif
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) g[v] = k3_ld16(gamma + k3_vec_off(t, v));
#if K3_PUSH == 3
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_add2_vec(pv[v], a[v], e[v], two);
#endif
    const float r = k3_row_rscale(k3_block_sum128(k3_row_sumsq(pv), s_red0, t), K3_PUSH_EPS);
#if K3_PUSH == 3
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) k3_st16(hidden + row + k3_vec_off(t, v), pv[v]);
#endif
    if (snapshot) {
#pragma unroll
      for (int v = 0; v < K3_KVPT; ++v)
        k3_st16_nt(blocks + (size_t)b * K3_NB_MAX * K3_H + k3_vec_off(t, v), pv[v]);
    }
    k3_u4 nv[K3_KVPT];
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        nv[v][j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(pv[v][j]) * r, k3_bf_hi(pv[v][j]) * r), g[v][j]);
    uint16_t* lrow = normed_all + dst_off;
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt(lrow + k3_vec_off(t, v), nv[v]);
    if (dst_peer) {
#pragma unroll
      for (int q = 0; q < K3_MAX_RANKS; ++q) {
        if (q >= nr) break;
        if (q == rank) continue;
        uint16_t* prow = (uint16_t*)(uintptr_t)dst_peer[q] + dst_off;
#pragma unroll
        for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt_g(prow + k3_vec_off(t, v), nv[v]);
      }
    }
    return;
  }

  k3_u4 pv[K3_KVPT];
#if K3_PUSH == 3
  k3_push_land_add2(p1, p2, prefix2, hidden, two, row, t, pv);
#else
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_ld16_nt(prefix + row + k3_vec_off(t, v));
#endif
  if (snapshot && nb < K3_NB_MAX) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v)
      k3_st16_nt(blocks + ((size_t)b * K3_NB_MAX + nb) * K3_H + k3_vec_off(t, v), pv[v]);
  }
  const K3NormedDst dst = {normed_all + dst_off, dst_peer, dst_off, rank, nr};
#if K3_PUSH >= 2
  k3_attnres_rms_row_to<-1, K3_MIX_STATS_OUT>(blocks + (size_t)b * K3_NB_MAX * K3_H, pv, sw, gamma,
                                              dst, nb, K3_PUSH_EPS, t, sw_mlp,
                                              stats + (size_t)b * K3_NB_MAX * 2);
#else
  k3_attnres_rms_row_to<-1>(blocks + (size_t)b * K3_NB_MAX * K3_H, pv, sw, gamma, dst, nb,
                            K3_PUSH_EPS, t);
#endif
}

// ---------------------------------------------------------------- nb 0, wide
// Typed-call entry k3h_attnres_rms_push_nb0w896 for nb == 0 (the module's
// parameter list; block 896, grid B): lane `tid` owns the row's vector tid, so
// each lane has one store per destination in flight.  The row goes through LDS
// once: lanes 0-127 replay the per-thread sums of squares in the K1 ownership
// (thread t: vectors t + 128 v, v = 0..6, one fma chain) and the half-wave
// partials in order, so r has the bits of the 128-thread body.  gamma is
// loaded ahead of the row, so the one wait for the row covers it, and the
// snapshot slot (and, for push_add2, `hidden`) is stored before the reduction.
// Measured at B 4096, 4 ranks (every normed copy local), back to back over 4
// rotating sets of buffers: 56.1 us (6.28 TB/s) against 69.2 for the module
// entry's 128-thread body, 60.1 with the snapshot stored after the reduction,
// 66.9 at 448 threads (2 vectors per lane); the same byte shape with no
// arithmetic runs 53.2 us at 896 threads and 71.2 at 128.
template <int NT>
K3_DEV void k3w_push_nb0(
#if K3_PUSH != 3
    const uint16_t* __restrict__ prefix,
#endif
    uint16_t* __restrict__ blocks, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ normed_all, const unsigned long long* __restrict__ dst_peer,
    int snapshot, int B, int rank, int nranks
#if K3_PUSH == 3
    , const uint16_t* __restrict__ p1, const uint16_t* __restrict__ p2,
    const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden, int two
#endif
) {
  constexpr int NV = 896 / NT;
  static_assert(NV * NT == 896 && NT >= K3_RES_THREADS, "NT divides the row's 896 vectors");
  __shared__ k3_u4 s_row[896];
  __shared__ float s_red[K3_NHW];
  const int b = blockIdx.x;
  if (b >= B) return;
  const int tid = threadIdx.x;
  const int nr = nranks < K3_MAX_RANKS ? nranks : K3_MAX_RANKS;
  const long long dst_off = ((long long)rank * B + b) * K3_H;
  const size_t row = (size_t)b * K3_H;
  k3_u4 pv[NV], g[NV];
  // gamma first: the wait for the row's own loads then covers it, and no
  // store issued after that wait is waited for again
#pragma unroll
  for (int v = 0; v < NV; ++v) g[v] = k3_ld16(gamma + (tid + NT * v) * 8);
  __builtin_amdgcn_sched_barrier(0);
#if K3_PUSH == 3
  k3_u4 a[NV], e[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    a[v] = k3_ld16_nt(p1 + row + (tid + NT * v) * 8);
    pv[v] = k3_ld16_nt(prefix2 + row + (tid + NT * v) * 8);
  }
  if (two) {
#pragma unroll
    for (int v = 0; v < NV; ++v) e[v] = k3_ld16_nt(p2 + row + (tid + NT * v) * 8);
  }
#else
#pragma unroll
  for (int v = 0; v < NV; ++v) pv[v] = k3_ld16_nt(prefix + row + (tid + NT * v) * 8);
#endif
#if K3_PUSH == 3
#pragma unroll
  for (int v = 0; v < NV; ++v) pv[v] = k3_add2_vec(pv[v], a[v], e[v], two);
#endif
#pragma unroll
  for (int v = 0; v < NV; ++v) s_row[tid + NT * v] = pv[v];
  // the rows that need neither r nor gamma leave before the reduction
  uint16_t* snap = snapshot ? blocks + (size_t)b * K3_NB_MAX * K3_H : nullptr;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#if K3_PUSH == 3
    k3_st16(hidden + row + (tid + NT * v) * 8, pv[v]);
#endif
    if (snap) k3_st16_nt(snap + (tid + NT * v) * 8, pv[v]);
  }
  __syncthreads();
  if (tid < K3_RES_THREADS) {
    k3_u4 kv[K3_KVPT];
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) kv[v] = s_row[tid + K3_RES_THREADS * v];
    const float part = k3_sum32(k3_row_sumsq(kv));
    if ((tid & 31) == 0) s_red[tid >> 5] = part;
  }
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < K3_NHW; ++w) tot += s_red[w];
  const float r = k3_row_rscale(tot, K3_PUSH_EPS);
  uint16_t* lrow = normed_all + dst_off;
  k3_u4 nv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      nv[v][j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(pv[v][j]) * r, k3_bf_hi(pv[v][j]) * r), g[v][j]);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int u = (tid + NT * v) * 8;
    k3_st16_nt(lrow + u, nv[v]);
    if (dst_peer) {
#pragma unroll
      for (int q = 0; q < K3_MAX_RANKS; ++q) {
        if (q >= nr) break;
        if (q == rank) continue;
        k3_st16_nt_g((uint16_t*)(uintptr_t)dst_peer[q] + dst_off + u, nv[v]);
      }
    }
  }
}

// ---------------------------------------------------------------- split form
template <int NB>
K3_DEV void k3s_push_body(
#if K3_PUSH != 3
    const uint16_t* __restrict__ prefix,
#endif
    uint16_t* __restrict__ blocks, const float* __restrict__ sw,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ normed_all,
    const unsigned long long* __restrict__ dst_peer, int snapshot, int B, int rank, int nranks
#if K3_PUSH >= 2
    , const float* __restrict__ sw_mlp, float* __restrict__ stats
#endif
#if K3_PUSH == 3
    , const uint16_t* __restrict__ p1, const uint16_t* __restrict__ p2,
    const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden, int two
#endif
) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const K3sLane L = k3s_lane();
  const int nr = nranks < K3_MAX_RANKS ? nranks : K3_MAX_RANKS;
  const long long dst_off = ((long long)rank * B + b) * K3_H;
  const size_t row = (size_t)b * K3_H;
  // every load of the row (the prefix or its land_add2 operands, the candidates)
  // goes out before the first store
  k3_u4 pv[K3S_SLOTS];
#if K3_PUSH == 3
  k3_u4 a[K3S_SLOTS], e[K3S_SLOTS];
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    a[s] = k3_ld16_nt(p1 + row + L.off(s));
    pv[s] = k3_ld16_nt(prefix2 + row + L.off(s));
  }
  if (two) {
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) e[s] = k3_ld16_nt(p2 + row + L.off(s));
  }
#else
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) pv[s] = k3_ld16_nt(prefix + row + L.off(s));
#endif
  k3_u4 xc[NB][K3S_SLOTS];
  k3s_load_candidates<NB>(xc, blocks + (size_t)b * K3_NB_MAX * K3_H, L);
  // hidden (K3_PUSH 3) and the snapshot slot are stored by the row body once
  // its own loads are out
  const K3NormedDst dst = {normed_all + dst_off, dst_peer, dst_off, rank, nr};
  const K3sPvStores pvst = {
#if K3_PUSH == 3
      hidden + row,
#else
      nullptr,
#endif
      snapshot && NB < K3_NB_MAX ? blocks + ((size_t)b * K3_NB_MAX + NB) * K3_H : nullptr,
      nullptr};
#if K3_PUSH == 3
  // the land_add2 sum runs after the body has issued its own loads (measured
  // equal to running it first, nb 4 at B 4096)
  k3s_attnres_rms_row<NB, K3_MIX_STATS_OUT>(xc, pv, sw, gamma, dst, pvst, K3_PUSH_EPS, L, nullptr,
                                             0, sw_mlp, stats + (size_t)b * K3_NB_MAX * 2,
                                             [&](k3_u4* p) {
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) p[s] = k3_add2_vec(p[s], a[s], e[s], two);
  });
#elif K3_PUSH == 2
  k3s_attnres_rms_row<NB, K3_MIX_STATS_OUT>(xc, pv, sw, gamma, dst, pvst, K3_PUSH_EPS, L, nullptr,
                                             0, sw_mlp, stats + (size_t)b * K3_NB_MAX * 2);
#else
  k3s_attnres_rms_row<NB, 0>(xc, pv, sw, gamma, dst, pvst, K3_PUSH_EPS, L, nullptr, 0);
#endif
}

#if K3_PUSH == 3
#define K3P_PARAMS                                                                          \
  uint16_t *__restrict__ blocks, const float *__restrict__ sw,                              \
      const uint16_t *__restrict__ gamma, uint16_t *__restrict__ normed_all,                \
      const unsigned long long *__restrict__ dst_peer, int nb, int snapshot, int B, int rank, \
      int nranks, const float *__restrict__ sw_mlp, float *__restrict__ stats,              \
      const uint16_t *__restrict__ p1, const uint16_t *__restrict__ p2,                     \
      const uint16_t *__restrict__ prefix2, uint16_t *__restrict__ hidden, int two
#define K3P_ARGS blocks, sw, gamma, normed_all, dst_peer, snapshot, B, rank, nranks, sw_mlp, \
                 stats, p1, p2, prefix2, hidden, two
#elif K3_PUSH == 2
#define K3P_PARAMS                                                                          \
  const uint16_t *__restrict__ prefix, uint16_t *__restrict__ blocks,                       \
      const float *__restrict__ sw, const uint16_t *__restrict__ gamma,                     \
      uint16_t *__restrict__ normed_all, const unsigned long long *__restrict__ dst_peer,    \
      int nb, int snapshot, int B, int rank, int nranks, const float *__restrict__ sw_mlp,  \
      float *__restrict__ stats
#define K3P_ARGS prefix, blocks, sw, gamma, normed_all, dst_peer, snapshot, B, rank, nranks, \
                 sw_mlp, stats
#else
#define K3P_PARAMS                                                                          \
  const uint16_t *__restrict__ prefix, uint16_t *__restrict__ blocks,                       \
      const float *__restrict__ sw, const uint16_t *__restrict__ gamma,                     \
      uint16_t *__restrict__ normed_all, const unsigned long long *__restrict__ dst_peer,    \
      int nb, int snapshot, int B, int rank, int nranks
#define K3P_ARGS prefix, blocks, sw, gamma, normed_all, dst_peer, snapshot, B, rank, nranks
#endif

// nb is the entry's K (the typed call checks it); the parameter keeps the
// module entry's list.
#define K3P_SPLIT_ENTRY(K)                                                                    \
  extern "C" __global__ void __launch_bounds__(K3S_THREADS)                                   \
      k3h_attnres_rms_push_nb##K##s(K3P_PARAMS) {                                             \
    (void)nb;                                                                                 \
    k3s_push_body<K>(K3P_ARGS);                                                               \
  }
K3P_SPLIT_ENTRY(1)
K3P_SPLIT_ENTRY(2)
K3P_SPLIT_ENTRY(3)
K3P_SPLIT_ENTRY(4)
K3P_SPLIT_ENTRY(5)
K3P_SPLIT_ENTRY(6)
K3P_SPLIT_ENTRY(7)
K3P_SPLIT_ENTRY(8)

#if K3_PUSH == 3
#define K3W_ARGS blocks, gamma, normed_all, dst_peer, snapshot, B, rank, nranks, p1, p2, prefix2, hidden, two
#else
#define K3W_ARGS prefix, blocks, gamma, normed_all, dst_peer, snapshot, B, rank, nranks
#endif
#define K3W_ENTRY(NT)                                                                         \
  extern "C" __global__ void __launch_bounds__(NT) k3h_attnres_rms_push_nb0w##NT(K3P_PARAMS) { \
    (void)nb; (void)sw;                                                                       \
    k3w_push_nb0<NT>(K3W_ARGS);                                                               \
  }
K3W_ENTRY(896)
