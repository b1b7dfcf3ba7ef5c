// K1 residual-stream row body for gfx950: AttnRes candidate mixing + RMSNorm of
// one 7168-wide bf16 row, computed by one 128-thread workgroup (two wave64s).
//
// Semantics follow the reference row body (k3_residual_v2.cu:107-257):
//   * candidates c < nb are rows blocks[b, c, :]; candidate nb is the prefix
//     row held in registers (pv);
//   * sq_c = sum x^2, dp_c = sum x * sw; score_c = dp_c * rsqrt(sq_c / H + eps);
//     p = softmax(score); mixed = bf16(sum_c p_c * x_c) in f32;
//   * r = rsqrt(sum mixed^2 / H + eps); normed = bf16(bf16(mixed * r) (x) gamma)
//     where (x) is the bf16 x bf16 -> bf16 product.
//
// Ownership and reduction order: thread t owns the 16-byte vectors
// u = t + 128 v (v < 7) of the row, i.e. elements 8u .. 8u + 7, so each wave
// issues 1 KB of contiguous loads per vector step.  Per-thread sums run over v
// (outer) and the eight elements (inner) with one fma each; a 32-lane xor
// butterfly follows inside each half-wave, and the four half-wave partials are
// added in half-wave order.  That is the order of the reference's 128-thread
// row (k3_residual_v2.cu:229-242), so the CPU checker can replay it exactly.
// rsqrt is 1 / sqrt with both operations correctly rounded; the softmax uses
// the deterministic k3_expf.  Both therefore have an exact CPU counterpart.
//
// Rows that are read or written once (partial, prefix, prefix2, normed) move
// with non-temporal loads and stores; gamma and sw stay cacheable.  Candidate
// rows: with one or two candidates (held in registers, read once) non-temporal;
// otherwise pass 1 reads them cacheable, so that pass 2 finds them in L2, and
// pass 2, their last use, reads them non-temporally (measured at B = 4096:
// nb 8 164 -> 151 us with a cold cache; cacheable everywhere, the loads also
// allocate in the MALL and, after a write-heavy predecessor, pay for evicting
// its dirty lines: nb 2 93 -> 70 us with non-temporal loads).
#pragma once
#include "../common/k3_dev.h"

#define K3_H 7168
#define K3_NB_MAX 8
#define K3_RES_THREADS 128
#define K3_KVPT 7                 /* 16-byte vectors per thread: 896 / 128 */
#define K3_NHW (K3_RES_THREADS / 32)  /* half-waves per workgroup */

#ifndef K3_EPS
#define K3_EPS 1e-5f
#endif

K3_DEV int k3_vec_off(int t, int v) { return (t + v * K3_RES_THREADS) * 8; }

// Sum of squares of this thread's vectors, reference order.
K3_DEV float k3_row_sumsq(const k3_u4* pv) {
  float sq = 0.0f;
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = k3_bf_lo(pv[v][j]), hi = k3_bf_hi(pv[v][j]);
      sq = __builtin_fmaf(lo, lo, sq);
      sq = __builtin_fmaf(hi, hi, sq);
    }
  }
  return sq;
}

// Block-wide total of a per-thread partial: half-wave butterfly, then the four
// half-wave partials added in order.  `red` is K3_NHW floats of LDS.  Ends with
// a barrier so `red` may be reused.
K3_DEV float k3_block_sum128(float part, float* red, int t) {
  part = k3_sum32(part);
  if ((t & 31) == 0) red[t >> 5] = part;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < K3_NHW; ++w) tot += red[w];
  __syncthreads();
  return tot;
}

// 1 / sqrt(sum / H + eps); the reference writes rsqrtf(sum * (1/H) + eps),
// which its compiler contracts into one fma.
K3_DEV float k3_row_rscale(float tot, float eps) {
  return k3_rsqrt_cr(__builtin_fmaf(tot, 1.0f / (float)K3_H, eps));
}

// AttnRes mixing: replaces pv (the prefix candidate) by the mixed row.
// NBC >= 0 fixes nb at compile time; NBC < 0 takes the run-time nb.
//
// MODE selects the candidate-statistics hand-off between the attention
// residual (res_in) and the MLP residual (res_mlp) of one layer
// (k3_residual_push_stats.cu:176-263, k3_residual_nb_stats.cu:176-258):
//   K3_MIX_STATS_OUT: for every block candidate c < nb also accumulate
//     dm_c = sum x * sw_mlp (same per-thread order and butterfly as dp_c) and
//     write stats_out[c] = (sq_c, dm_c), the half-wave-0 totals;
//   K3_MIX_STATS_IN: candidates c < ns = min(nb_stats, nb) take (sq_c, dp_c)
//     from stats_in[c] instead of reading their rows in pass 1 (pass 2 still
//     reads every candidate).  Given statistics produced by STATS_OUT with
//     sw_mlp equal to this call's sw, the result is bit-identical to MODE 0.
// stats rows are [K3_NB_MAX][2] floats.
#define K3_MIX_STATS_OUT 1
#define K3_MIX_STATS_IN 2
#define K3_MIX_NO_HOLD 4  /* keep no vector steps across the passes (register budget) */

// Zero that the compiler cannot see through, computed after `dep`.  Added to
// the addresses of a vector step's loads, it keeps them from being issued
// before the value they are made to wait for (with straight-line code the
// compiler otherwise hoists every step's loads to the top of the pass) and from
// being merged with identical loads of an earlier pass.
K3_DEV int k3_zero_after(float dep) {
  int z = 0;
  asm volatile("" : "+v"(z) : "v"(dep));
  return z;
}

template <int NBC, int MODE = 0>
K3_DEV void k3_attnres_mix(const uint16_t* __restrict__ blk_row, k3_u4* pv,
                           const float* __restrict__ sw, int nb_rt, float eps, int t,
                           const float* __restrict__ sw_mlp = nullptr,
                           float* __restrict__ stats_out = nullptr,
                           const float* __restrict__ stats_in = nullptr, int nb_stats = 0) {
  constexpr bool SOUT = (MODE & K3_MIX_STATS_OUT) != 0;
  constexpr bool SIN = (MODE & K3_MIX_STATS_IN) != 0;
  const int nb = NBC >= 0 ? NBC : nb_rt;
  if (nb <= 0) return;  // mixed = prefix: bf16(1.0f * f32(prefix)) == prefix
  const int ns = SIN ? (nb_stats < 0 ? 0 : nb_stats < nb ? nb_stats : nb) : 0;
  __shared__ float s_red[(K3_NB_MAX + 1) * 2 * K3_NHW];
  __shared__ float s_redm[SOUT ? K3_NB_MAX * K3_NHW : 1];
  const int lane32 = t & 31, hw = t >> 5;

  // pass 1: sum x^2 and sum x * sw per candidate (prefix kept at index K3_NB_MAX).
  // A vector step's loads (candidates, sw, sw_mlp) all go out before any use,
  // and the next step's loads go out before this step's arithmetic (the vector
  // memory counter retires in issue order, so a step's loads are issued
  // together and waited for together).
  // With one or two candidates (compile-time nb) the candidate rows stay in
  // registers from pass 1 to pass 2 (RES): all their loads go out first and
  // pass 2 reads nothing.
  // PF: vector steps whose loads are in flight beyond the current one (deeper
  // prefetch measured no faster: at nb >= 3 the time goes to pass 2 re-reading
  // candidates that no longer are in the 4 MB per-XCD L2).
  constexpr int PF = 1;
  constexpr bool RES = NBC >= 1 && NBC <= 2;
  k3_u4 xr[RES ? NBC : 1][K3_KVPT];
  // HOLD: with a compile-time nb >= 3 (and no statistics hand-off) the first
  // HOLD vector steps of every candidate stay in registers from pass 1 to pass 2;
  // pass 2 re-reads only the later steps, which pass 1 read last.  Measured at
  // B = 4096 (the nb entries): nb 5 165 -> 157 us, nb 8 207 -> 201 us, nb 3, 4, 6
  // within 1-2%, nb 7 none (the registers would push it to one wave per SIMD).
  constexpr int HOLD = (RES || SIN || (MODE & K3_MIX_NO_HOLD)) ? 0
                       : (NBC >= 3 && NBC <= 6) ? 2 : NBC == 8 ? 1 : 0;
  k3_u4 xh[HOLD > 0 ? HOLD : 1][K3_NB_MAX];
  if constexpr (RES) {
#pragma unroll
    for (int c = 0; c < NBC; ++c)
#pragma unroll
      for (int v = 0; v < K3_KVPT; ++v) xr[c][v] = k3_ld16_nt(blk_row + (size_t)c * K3_H + k3_vec_off(t, v));
  }
  float sq[K3_NB_MAX + 1], dp[K3_NB_MAX + 1], dm[K3_NB_MAX];
#pragma unroll
  for (int c = 0; c <= K3_NB_MAX; ++c) { sq[c] = 0.0f; dp[c] = 0.0f; }
#pragma unroll
  for (int c = 0; c < K3_NB_MAX; ++c) dm[c] = 0.0f;
  k3_u4 xb[PF + 1][K3_NB_MAX];
  float4 wb[PF + 1][SOUT ? 4 : 2];
  auto load1 = [&](int v, int slot, float dep) {
    const int u = k3_vec_off(t, v) + k3_zero_after(dep);
#pragma unroll
    for (int c = 0; c < K3_NB_MAX; ++c) {
      if (RES || c >= nb) break;
      if (SIN && c < ns) continue;
      xb[slot][c] = k3_ld16(blk_row + (size_t)c * K3_H + u);
    }
    wb[slot][0] = *(const float4*)(sw + u);
    wb[slot][1] = *(const float4*)(sw + u + 4);
    if (SOUT) {
      wb[slot][SOUT ? 2 : 0] = *(const float4*)(sw_mlp + u);
      wb[slot][SOUT ? 3 : 1] = *(const float4*)(sw_mlp + u + 4);
    }
  };
#pragma unroll
  for (int d = 0; d < PF; ++d) load1(d, d, __uint_as_float(pv[0][0]));
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    const int slot = v % (PF + 1);
    // the loads of step v + 1 wait for every sum of step v - 1: two steps in
    // flight at most
    float dep = dp[K3_NB_MAX];
#pragma unroll
    for (int c = 0; c < K3_NB_MAX; ++c) {
      if (c >= nb) break;
      dep += sq[c] + dp[c];
      if (SOUT) dep += dm[c];
    }
    if (v + PF < K3_KVPT) load1(v + PF, (v + PF) % (PF + 1), dep);
    const float4 a = wb[slot][0], b = wb[slot][1];
    const float swv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float swm[8];
    if (SOUT) {
      const float4 ma = wb[slot][SOUT ? 2 : 0], mb = wb[slot][SOUT ? 3 : 1];
      swm[0] = ma.x; swm[1] = ma.y; swm[2] = ma.z; swm[3] = ma.w;
      swm[4] = mb.x; swm[5] = mb.y; swm[6] = mb.z; swm[7] = mb.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = k3_bf_lo(pv[v][j]), hi = k3_bf_hi(pv[v][j]);
      sq[K3_NB_MAX] = __builtin_fmaf(lo, lo, sq[K3_NB_MAX]);
      sq[K3_NB_MAX] = __builtin_fmaf(hi, hi, sq[K3_NB_MAX]);
      dp[K3_NB_MAX] = __builtin_fmaf(lo, swv[2 * j], dp[K3_NB_MAX]);
      dp[K3_NB_MAX] = __builtin_fmaf(hi, swv[2 * j + 1], dp[K3_NB_MAX]);
    }
#pragma unroll
    for (int c = 0; c < K3_NB_MAX; ++c) {
      if (c >= nb) break;
      if (SIN && c < ns) continue;
      k3_u4 x;
      if constexpr (RES) x = xr[c][v];
      else x = xb[slot][c];
      if constexpr (HOLD > 0) {
        if (v < HOLD) xh[v < HOLD ? v : 0][c] = x;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = k3_bf_lo(x[j]), hi = k3_bf_hi(x[j]);
        sq[c] = __builtin_fmaf(lo, lo, sq[c]);
        sq[c] = __builtin_fmaf(hi, hi, sq[c]);
        dp[c] = __builtin_fmaf(lo, swv[2 * j], dp[c]);
        dp[c] = __builtin_fmaf(hi, swv[2 * j + 1], dp[c]);
        if (SOUT) {
          dm[c] = __builtin_fmaf(lo, swm[2 * j], dm[c]);
          dm[c] = __builtin_fmaf(hi, swm[2 * j + 1], dm[c]);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < K3_NB_MAX; ++c) {
    if (c >= nb) break;
    if (SIN && c < ns) continue;
    const float s = k3_sum32(sq[c]);
    const float d = k3_sum32(dp[c]);
    if (lane32 == 0) { s_red[(2 * c) * K3_NHW + hw] = s; s_red[(2 * c + 1) * K3_NHW + hw] = d; }
    if (SOUT) {
      const float m = k3_sum32(dm[c]);
      if (lane32 == 0) s_redm[c * K3_NHW + hw] = m;
    }
  }
  {
    const float s = k3_sum32(sq[K3_NB_MAX]);
    const float d = k3_sum32(dp[K3_NB_MAX]);
    if (lane32 == 0) { s_red[(2 * nb) * K3_NHW + hw] = s; s_red[(2 * nb + 1) * K3_NHW + hw] = d; }
  }
  __syncthreads();

  // scores and softmax: lane c of every half-wave handles candidate c
  const int ncand = nb + 1;
  float sc = -3.0e38f;
  if (lane32 < ncand) {
    float sqv = 0.0f, dpv = 0.0f;
    if (SIN && lane32 < ns) {
      sqv = stats_in[2 * lane32];
      dpv = stats_in[2 * lane32 + 1];
    } else {
#pragma unroll
      for (int w = 0; w < K3_NHW; ++w) {
        sqv += s_red[(2 * lane32) * K3_NHW + w];
        dpv += s_red[(2 * lane32 + 1) * K3_NHW + w];
      }
    }
    if (SOUT && hw == 0 && lane32 < nb) {
      float dmv = 0.0f;
#pragma unroll
      for (int w = 0; w < K3_NHW; ++w) dmv += s_redm[lane32 * K3_NHW + w];
      stats_out[2 * lane32] = sqv;
      stats_out[2 * lane32 + 1] = dmv;
    }
    sc = dpv * k3_row_rscale(sqv, eps);
  }
  const float mx = k3_max32(sc);
  float ex = 0.0f;
  if (lane32 < ncand) {
    const float d = sc - mx;
    ex = d < -87.0f ? 0.0f : k3_expf(d);
  }
  const float den = k3_sum32(ex);
  const float pmine = ex / den;
  const int base = t & 32;  // lanes of this half-wave within the wave
  float p[K3_NB_MAX];
#pragma unroll
  for (int c = 0; c < K3_NB_MAX; ++c) p[c] = __shfl(pmine, base + c, 64);
  const float pp = __shfl(pmine, base + nb, 64);

  // pass 2: f32 mix, one bf16 landing per value (loads issued as in pass 1).
  // The row base goes through an empty asm so that the compiler re-loads the
  // candidates here instead of keeping every pass-1 value live across the
  // softmax (7 nb vectors per thread: more registers than a wave has at nb >= 3).
  auto load2 = [&](int v, int slot, float dep) {
    const int u = k3_vec_off(t, v) + k3_zero_after(dep);
#pragma unroll
    for (int c = 0; c < K3_NB_MAX; ++c) {
      if (RES || c >= nb) break;
      xb[slot][c] = k3_ld16_nt(blk_row + (size_t)c * K3_H + u);
    }
  };
  // Pass 2 walks the vectors last-read-first: the candidates pass 1 touched last
  // are the likeliest still in L2 (each value's sum is independent of v).
  float dep2 = pp;
#pragma unroll
  for (int d = 0; d < PF; ++d) load2(K3_KVPT - 1 - d, d, dep2);
#pragma unroll
  for (int w = 0; w < K3_KVPT; ++w) {
    const int v = K3_KVPT - 1 - w;
    const int slot = w % (PF + 1);
    if (w + PF < K3_KVPT && v - PF >= HOLD) load2(v - PF, (w + PF) % (PF + 1), dep2);
    const k3_u4* xv = xb[slot];
    float acc[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = pp * k3_bf_lo(pv[v][j]);
      acc[2 * j + 1] = pp * k3_bf_hi(pv[v][j]);
    }
#pragma unroll
    for (int c = 0; c < K3_NB_MAX; ++c) {
      if (c >= nb) break;
      k3_u4 x;
      if constexpr (RES) x = xr[c][v];
      else if (HOLD > 0 && v < HOLD) x = xh[v < HOLD ? v : 0][c];
      else x = xv[c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = __builtin_fmaf(p[c], k3_bf_lo(x[j]), acc[2 * j]);
        acc[2 * j + 1] = __builtin_fmaf(p[c], k3_bf_hi(x[j]), acc[2 * j + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) pv[v][j] = k3_pack_bf2(acc[2 * j], acc[2 * j + 1]);
    dep2 = __uint_as_float(pv[v][0] ^ pv[v][1] ^ pv[v][2] ^ pv[v][3]);
  }
}

// normed = bf16(bf16(mixed * r) (x) gamma) for this thread's vectors; returns
// the normed vectors in `nv`.
K3_DEV void k3_rms_apply(const k3_u4* pv, const uint16_t* __restrict__ gamma, float r,
                         k3_u4* nv, int t) {
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    const k3_u4 g = k3_ld16(gamma + k3_vec_off(t, v));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t y = k3_pack_bf2(k3_bf_lo(pv[v][j]) * r, k3_bf_hi(pv[v][j]) * r);
      nv[v][j] = k3_mul_bf2(y, g[j]);
    }
  }
}

// Where a row body stores its normed row: `row`, and, for the push entries, the
// same row offset `off` of every other rank's buffer peer[q], q < nr, q != rank
// (k3_residual_push_v3.cu:306-312).  peer == nullptr: the local row only.
#define K3_MAX_RANKS 8
struct K3NormedDst {
  uint16_t* row;
  const unsigned long long* peer;
  long long off;
  int rank, nr;
};

// The whole row body: mixing (if any), RMS, normed store(s).  MODE, sw_mlp and
// the stats arguments are those of k3_attnres_mix.
template <int NBC, int MODE = 0>
K3_DEV void k3_attnres_rms_row_to(const uint16_t* __restrict__ blk_row, k3_u4* pv,
                                  const float* __restrict__ sw, const uint16_t* __restrict__ gamma,
                                  const K3NormedDst& dst, int nb, float eps, int t,
                                  const float* __restrict__ sw_mlp = nullptr,
                                  float* __restrict__ stats_out = nullptr,
                                  const float* __restrict__ stats_in = nullptr, int nb_stats = 0) {
#ifndef K3_NB_SWITCH
#define K3_NB_SWITCH 1
#endif
  if constexpr (NBC < 0 && K3_NB_SWITCH) {
    // run-time nb: branch once (uniformly) into the compile-time instantiation,
    // which drops the unused candidate registers and guards and keeps one or two
    // candidates resident (no held vector steps: every instantiation shares the
    // kernel's register budget)
#define K3_NB_CASE(K)                                                                         \
  case K:                                                                                     \
    k3_attnres_rms_row_to<K, MODE | K3_MIX_NO_HOLD>(blk_row, pv, sw, gamma, dst, K, eps, t,   \
                                                    sw_mlp, stats_out, stats_in, nb_stats);   \
    return;
    switch (nb) {
      K3_NB_CASE(0) K3_NB_CASE(1) K3_NB_CASE(2) K3_NB_CASE(3) K3_NB_CASE(4)
      K3_NB_CASE(5) K3_NB_CASE(6) K3_NB_CASE(7) K3_NB_CASE(8)
      default:
        break;
    }
#undef K3_NB_CASE
  }
  __shared__ float s_red2[K3_NHW];
  k3_attnres_mix<NBC, MODE>(blk_row, pv, sw, nb, eps, t, sw_mlp, stats_out, stats_in, nb_stats);
  const float tot = k3_block_sum128(k3_row_sumsq(pv), s_red2, t);
  const float r = k3_row_rscale(tot, eps);
  k3_u4 nv[K3_KVPT];
  k3_rms_apply(pv, gamma, r, nv, t);
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt(dst.row + k3_vec_off(t, v), nv[v]);
  if (dst.peer) {
#pragma unroll
    for (int q = 0; q < K3_MAX_RANKS; ++q) {
      if (q >= dst.nr) break;
      if (q == dst.rank) continue;
      uint16_t* prow = (uint16_t*)(uintptr_t)dst.peer[q] + dst.off;
#pragma unroll
      for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt_g(prow + k3_vec_off(t, v), nv[v]);
    }
  }
}

template <int NBC>
K3_DEV void k3_attnres_rms_row(const uint16_t* __restrict__ blk_row, k3_u4* pv,
                               const float* __restrict__ sw, const uint16_t* __restrict__ gamma,
                               uint16_t* __restrict__ normed_row, int nb, float eps, int t) {
  const K3NormedDst dst = {normed_row, nullptr, 0, 0, 1};
  k3_attnres_rms_row_to<NBC>(blk_row, pv, sw, gamma, dst, nb, eps, t);
}

// K1b landing: prefix2 = snapshot ? bf16(pf) : bf16(f32(prefix) + f32(bf16(pf))).
// LAND_BF16 = partial arrives as bf16 (bf16(pf) == pf); otherwise f32.
#ifdef LAND_BF16
typedef uint16_t k3_land_t;
#else
typedef float k3_land_t;
#endif

K3_DEV k3_u4 k3_load_land(const k3_land_t* __restrict__ partial, size_t off) {
#ifdef LAND_BF16
  return k3_ld16_nt(partial + off);
#else
  const float4 a = k3_ld16f_nt(partial + off);
  const float4 c = k3_ld16f_nt(partial + off + 4);
  k3_u4 w;
  w[0] = k3_pack_bf2(a.x, a.y);
  w[1] = k3_pack_bf2(a.z, a.w);
  w[2] = k3_pack_bf2(c.x, c.y);
  w[3] = k3_pack_bf2(c.z, c.w);
  return w;
#endif
}

K3_DEV k3_u4 k3_add_land(k3_u4 prefix, k3_u4 landed) {
  k3_u4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = k3_pack_bf2(k3_bf_lo(prefix[j]) + k3_bf_lo(landed[j]),
                       k3_bf_hi(prefix[j]) + k3_bf_hi(landed[j]));
  return o;
}

// K1b row without candidates (nb == 0): every load first (the landing operands
// and gamma), the reduction, then the prefix2 and normed stores, so that no load
// waits behind a store (the vector memory counter retires in order).  Same
// arithmetic as the general body at nb == 0.
K3_DEV void k3_land_add_rms_nb0(const k3_land_t* __restrict__ partial,
                                const uint16_t* __restrict__ prefix,
                                const uint16_t* __restrict__ gamma,
                                uint16_t* __restrict__ prefix2, uint16_t* __restrict__ normed,
                                int snapshot, int b, int t, float eps) {
  __shared__ float s_red0[K3_NHW];
  k3_u4 pv[K3_KVPT], pr[K3_KVPT], g[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_load_land(partial, (size_t)b * K3_H + k3_vec_off(t, v));
  if (!snapshot) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pr[v] = k3_ld16_nt(prefix + (size_t)b * K3_H + k3_vec_off(t, v));
  }
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) g[v] = k3_ld16(gamma + k3_vec_off(t, v));
  if (!snapshot) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_add_land(pr[v], pv[v]);
  }
  const float tot = k3_block_sum128(k3_row_sumsq(pv), s_red0, t);
  const float r = k3_row_rscale(tot, eps);
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt(prefix2 + (size_t)b * K3_H + k3_vec_off(t, v), pv[v]);
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) {
    k3_u4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t y = k3_pack_bf2(k3_bf_lo(pv[v][j]) * r, k3_bf_hi(pv[v][j]) * r);
      o[j] = k3_mul_bf2(y, g[v][j]);
    }
    k3_st16_nt(normed + (size_t)b * K3_H + k3_vec_off(t, v), o);
  }
}

// K1b entry body shared by the run-time-nb entry and the per-nb entries.  With
// MODE = K3_MIX_STATS_IN the first nb_stats candidates' statistics come from
// stats[b] ([B, K3_NB_MAX, 2], written by the push-stats entry of res_in).
template <int NBC, int MODE = 0>
K3_DEV void k3_land_add_attnres_rms_body(const k3_land_t* __restrict__ partial,
                                         const uint16_t* __restrict__ prefix,
                                         const uint16_t* __restrict__ blocks,
                                         const float* __restrict__ sw,
                                         const uint16_t* __restrict__ gamma,
                                         uint16_t* __restrict__ prefix2,
                                         uint16_t* __restrict__ normed, int nb, int snapshot, int B,
                                         const float* __restrict__ stats = nullptr,
                                         int nb_stats = 0) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const int t = threadIdx.x;
  if (NBC <= 0 && nb == 0) {
    k3_land_add_rms_nb0(partial, prefix, gamma, prefix2, normed, snapshot, b, t, K3_EPS);
    return;
  }
  // all row loads first, then the landing adds and the prefix2 stores (a store
  // between two loads would make the second load's wait cover the store too)
  k3_u4 pv[K3_KVPT], pr[K3_KVPT];
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_load_land(partial, (size_t)b * K3_H + k3_vec_off(t, v));
  if (!snapshot) {
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pr[v] = k3_ld16_nt(prefix + (size_t)b * K3_H + k3_vec_off(t, v));
#pragma unroll
    for (int v = 0; v < K3_KVPT; ++v) pv[v] = k3_add_land(pr[v], pv[v]);
  }
#pragma unroll
  for (int v = 0; v < K3_KVPT; ++v) k3_st16_nt(prefix2 + (size_t)b * K3_H + k3_vec_off(t, v), pv[v]);
  const K3NormedDst dst = {normed + (size_t)b * K3_H, nullptr, 0, 0, 1};
  const bool have_stats = MODE != 0 && stats != nullptr;  // no statistics: nb_stats acts as 0
  k3_attnres_rms_row_to<NBC, MODE>(blocks + (size_t)b * K3_NB_MAX * K3_H, pv, sw, gamma, dst, nb,
                                   K3_EPS, t, nullptr, nullptr,
                                   have_stats ? stats + (size_t)b * K3_NB_MAX * 2 : nullptr,
                                   have_stats ? nb_stats : 0);
}
