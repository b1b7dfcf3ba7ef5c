// Module k3_residual_nb+LAND_BF16=1: K1b with the candidate count fixed per entry.
//
//   kern_k3_land_add_attnres_rms_nb{1..8}(partial, prefix, blocks, sw, gamma,
//                                         prefix2, normed, nb_in, snapshot, B)
//
// Same parameters, geometry (grid (B,1,1), block 128) and arithmetic as
// kern_k3_land_add_attnres_rms; the entry for k returns at once unless
// nb_in == k (reference: k3_residual_nb.cu:350-811).  Fixing nb lets the
// compiler drop the unused candidate registers.
//
// Module k3_residual_nb_stats (K3_NB_STATS and LAND_BF16, implied by the base
// name): the same entries with two more parameters,
//
//   kern_k3_land_add_attnres_rms_nb{1..8}(..., nb_in, snapshot, B, stats, nb_stats)
//
// where the first nb_stats candidates' (sum x^2, sum x * sw) come from
// stats[b] ([B, 8, 2] f32, written by res_in's push-stats entry) instead of a
// pass over their rows (k3_residual_nb_stats.cu:176-258, 366-811; manifest ops
// land_add_attnres_rms_bf16_v2_nb4..8).  nb_stats is clamped to [0, nb].
#include "k3_residual_split.h"

#ifndef K3_NB_STATS
#define K3_NB_ENTRY(K)                                                                      \
  extern "C" __global__ void __launch_bounds__(K3_RES_THREADS)                              \
      kern_k3_land_add_attnres_rms_nb##K(                                                   \
          const k3_land_t* __restrict__ partial, const uint16_t* __restrict__ prefix,       \
          const uint16_t* __restrict__ blocks, const float* __restrict__ sw,                \
          const uint16_t* __restrict__ gamma, uint16_t* __restrict__ prefix2,               \
          uint16_t* __restrict__ normed, int nb_in, int snapshot, int B) {                  \
    if (nb_in != K) return;                                                                 \
    k3_land_add_attnres_rms_body<K>(partial, prefix, blocks, sw, gamma, prefix2, normed, K, \
                                    snapshot, B);                                           \
  }
#else
#define K3_NB_ENTRY(K)                                                                        \
  extern "C" __global__ void __launch_bounds__(K3_RES_THREADS)                                \
      kern_k3_land_add_attnres_rms_nb##K(                                                     \
          const k3_land_t* __restrict__ partial, const uint16_t* __restrict__ prefix,         \
          const uint16_t* __restrict__ blocks, const float* __restrict__ sw,                  \
          const uint16_t* __restrict__ gamma, uint16_t* __restrict__ prefix2,                 \
          uint16_t* __restrict__ normed, int nb_in, int snapshot, int B,                      \
          const float* __restrict__ stats, int nb_stats) {                                    \
    if (nb_in != K) return;                                                                   \
    k3_land_add_attnres_rms_body<K, K3_MIX_STATS_IN>(partial, prefix, blocks, sw, gamma,      \
                                                     prefix2, normed, K, snapshot, B, stats, \
                                                     nb_stats);                               \
  }
#endif

// Typed-call entries with no reference counterpart: the same contract on the
// vector-split row body (k3_residual_split.h), grid (B, 1, 1), block 256:
//   k3h_land_add_attnres_rms_nb{1..8}s(..., nb_in, snapshot, B[, stats, nb_stats])
// Measured at B = 4096 with cold caches, against the 128-thread entries (HIP
// events, median): nb 1 / 4 / 6 / 8 59.1 / 98.1 / 120.3 / 151.8 -> 58.4 / 85.1 /
// 109.0 / 131.0 us; after a dirty-cache flush the 128-thread entries, whose
// pass 2 re-reads candidates through the caches, take 131.9 / 160.4 / 186.6 us
// at nb 4 / 6 / 8 and the split ones 85.1 / 106.2 / 127.6.
#ifndef K3_NB_STATS
#define K3_NBS_ENTRY(K)                                                                     \
  extern "C" __global__ void __launch_bounds__(K3S_THREADS)                              \
      k3h_land_add_attnres_rms_nb##K##s(                                                    \
          const k3_land_t* __restrict__ partial, const uint16_t* __restrict__ prefix,       \
          const uint16_t* __restrict__ blocks, const float* __restrict__ sw,                \
          const uint16_t* __restrict__ gamma, uint16_t* __restrict__ prefix2,               \
          uint16_t* __restrict__ normed, int nb_in, int snapshot, int B) {                  \
    if (nb_in != K) return;                                                                 \
    k3s_land_add_attnres_rms_body<K>(partial, prefix, blocks, sw, gamma, prefix2, normed,   \
                                     snapshot, B);                                          \
  }
#else
#define K3_NBS_ENTRY(K)                                                                     \
  extern "C" __global__ void __launch_bounds__(K3S_THREADS)                              \
      k3h_land_add_attnres_rms_nb##K##s(                                                    \
          const k3_land_t* __restrict__ partial, const uint16_t* __restrict__ prefix,       \
          const uint16_t* __restrict__ blocks, const float* __restrict__ sw,                \
          const uint16_t* __restrict__ gamma, uint16_t* __restrict__ prefix2,               \
          uint16_t* __restrict__ normed, int nb_in, int snapshot, int B,                    \
          const float* __restrict__ stats, int nb_stats) {                                  \
    if (nb_in != K) return;                                                                 \
    k3s_land_add_attnres_rms_body<K, K3_MIX_STATS_IN>(partial, prefix, blocks, sw, gamma,   \
                                                      prefix2, normed, snapshot, B, stats, \
                                                      nb_stats);                            \
  }
#endif

K3_NBS_ENTRY(1)
K3_NBS_ENTRY(2)
K3_NBS_ENTRY(3)
K3_NBS_ENTRY(4)
K3_NBS_ENTRY(5)
K3_NBS_ENTRY(6)
K3_NBS_ENTRY(7)
K3_NBS_ENTRY(8)

K3_NB_ENTRY(1)
K3_NB_ENTRY(2)
K3_NB_ENTRY(3)
K3_NB_ENTRY(4)
K3_NB_ENTRY(5)
K3_NB_ENTRY(6)
K3_NB_ENTRY(7)
K3_NB_ENTRY(8)
