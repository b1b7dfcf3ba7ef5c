// K1 row body, vector-split form: the AttnRes mix + RMSNorm of one 7168-wide
// bf16 row (the semantics of k3_residual_row.h, k3_residual_v2.cu:107-257) on
// 256 threads, with every candidate row held in registers from pass 1 to pass 2.
//
// Each reference thread rt (owner of the 16-byte vectors rt + 128 v, v < 7) is
// played by two lanes of one wave: rt = 32 w + (lane & 31) for wave w < 4, and
// half h = lane / 32 owns the vector steps v = 4 h + s, s < 4 (half 0: v 0..3,
// half 1: v 4..6; its fourth slot does not exist -- its loads repeat v = 6 and
// its results are never used or stored).  Half the vector steps per lane halves
// the registers a candidate takes, so all nb + 1 candidates of the row stay on
// chip and pass 2 reads nothing.
//
// The reference's sums are serial over v within a thread.  They are kept bit
// for bit by handing the chains over: every lane first runs the chain over its
// slots 0..3 from zero (half 0's result is then the reference thread's sum over
// v 0..3), half 1 takes half 0's partial sums (one lane shuffle per sum), and
// continues the chain over its slots 0..2 (v 4..6).  Half 1 then holds the
// reference thread's sums; the 32-lane butterfly and the four per-wave partials
// (in wave order) follow as in the 128-thread body.  The pass-2 mix is
// element-wise (its chain runs over candidates), so each lane mixes its own
// slots.  The RMS of the mixed row uses the same chain hand-over.
//
// Registers decide the speed: at nb 8 the held rows take 128 of a lane's
// registers, and two waves per SIMD (at most 256 registers) must fit.  Each run
// over the slots therefore unpacks the held bf16 rows afresh, slot by slot
// (empty asm statements make the packed rows the only live copy), instead of
// keeping the unpacked floats of one run alive into the next: 408 -> 208
// registers at nb 8 (1 -> 2 waves per SIMD), 209 -> 147 at nb 4 (2 -> 3).
// The prefix-row stores (prefix2, hidden, the snapshot slot) follow the row
// body's own loads (sw, sw_mlp, gamma): no load waits behind a store.
//
// Launch: block 256, one row per workgroup (grid B).  No reference entry uses
// this geometry; the manifest entries keep the 128-thread body.
#pragma once
#include "k3_residual_row.h"

#define K3S_THREADS 256
#define K3S_SLOTS 4

struct K3sLane {
  int w, lane, h, rt;
  K3_DEV int v(int s) const { return 4 * h + s; }
  K3_DEV bool valid(int s) const { return 4 * h + s < K3_KVPT; }
  // element offset of slot s in the row (the missing step re-reads step 6)
  K3_DEV int off(int s) const {
    const int vv = 4 * h + s < K3_KVPT ? 4 * h + s : K3_KVPT - 1;
    return (rt + K3_RES_THREADS * vv) * 8;
  }
};

K3_DEV K3sLane k3s_lane() {
  K3sLane L;
  L.w = threadIdx.x >> 6;
  L.lane = threadIdx.x & 63;
  L.h = L.lane >> 5;
  L.rt = 32 * L.w + (L.lane & 31);
  return L;
}

// Half 1 takes half 0's value (half 0 gets half 1's, which it never uses).
K3_DEV float k3s_handover(float v) { return __shfl_xor(v, 32, 64); }

// sum x^2 of the lane's slots s < n, continuing from `acc` (reference order:
// step outer, element inner, one fma each)
K3_DEV float k3s_sumsq(const k3_u4* x, int n, float acc) {
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    if (s >= n) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = k3_bf_lo(x[s][j]), hi = k3_bf_hi(x[s][j]);
      acc = __builtin_fmaf(lo, lo, acc);
      acc = __builtin_fmaf(hi, hi, acc);
    }
  }
  return acc;
}

// Row total of a per-reference-thread chain: run over slots 0..3, hand half 0's
// partial to half 1, run half 1's slots 0..2, butterfly, per-wave partials in
// wave order.  `red` is 4 floats of LDS; ends with a barrier.
K3_DEV float k3s_row_sumsq_total(const k3_u4* x, float* red, const K3sLane& L) {
  float a = k3s_sumsq(x, K3S_SLOTS, 0.0f);
  a = k3s_sumsq(x, K3_KVPT - K3S_SLOTS, k3s_handover(a));
  a = k3_sum32(a);
  if (L.lane == 32) red[L.w] = a;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) tot += red[w];
  __syncthreads();
  return tot;
}

// Stores of the prefix candidate (prefix2, hidden, the snapshot slot) that the
// row body issues once its own loads (sw, sw_mlp) are out, so that no load
// waits behind them (the vector memory counter retires in order and counts
// stores): `cached` goes through the caches, `nt0` and `nt1` are non-temporal.
struct K3sPvStores {
  uint16_t* cached;
  uint16_t* nt0;
  uint16_t* nt1;
};

// The mix + RMS of one row: pv holds the prefix candidate (the landed prefix2)
// for the lane's slots; candidates c < NB are read from blk_row.  MODE:
// 0, K3_MIX_STATS_IN (the first ns = min(nb_stats, NB) candidates take
// (sum x^2, sum x * sw) from stats_in, [K3_NB_MAX][2]) or K3_MIX_STATS_OUT (below).
// The candidate rows' loads of the lane's slots (each row is read once:
// non-temporal), issued by the caller before anything it stores.
template <int NB>
K3_DEV void k3s_load_candidates(k3_u4 (&xc)[NB][K3S_SLOTS], const uint16_t* __restrict__ blk_row,
                                const K3sLane& L) {
#pragma unroll
  for (int c = 0; c < NB; ++c)
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) xc[c][s] = k3_ld16_nt(blk_row + (size_t)c * K3_H + L.off(s));
}

// MODE also takes K3_MIX_STATS_OUT: every candidate c < NB also accumulates
// dm_c = sum x * sw_mlp (the same chain and butterfly as dp_c) and
// stats_out[c] = (sq_c, dm_c) is written (the 128-thread body's half-wave-0 totals:
// the four per-wave partials summed in wave order).  The normed row goes to every
// destination of `dst` (the local row and, for the push entries, each peer's).
// No step between the row body's own loads and its first use of pv.
struct K3sNoPre {
  K3_DEV void operator()(k3_u4*) const {}
};

// pre(pv) runs once the body's own loads (sw, sw_mlp, gamma) are issued: the
// callers that form the prefix row from landing operands do it there, so that
// those loads do not wait behind the operands' arrival.
template <int NB, int MODE, class Pre = K3sNoPre>
K3_DEV void k3s_attnres_rms_row(k3_u4 (&xc)[NB][K3S_SLOTS], k3_u4* pv,
                                const float* __restrict__ sw, const uint16_t* __restrict__ gamma,
                                const K3NormedDst& dst, const K3sPvStores& pvst, float eps,
                                const K3sLane& L, const float* __restrict__ stats_in,
                                int nb_stats, const float* __restrict__ sw_mlp = nullptr,
                                float* __restrict__ stats_out = nullptr, Pre pre = Pre()) {
  static_assert(NB >= 1 && NB <= K3_NB_MAX, "NB in 1..8");
  constexpr bool SIN = (MODE & K3_MIX_STATS_IN) != 0;
  constexpr bool SOUT = (MODE & K3_MIX_STATS_OUT) != 0;
  const int ns = SIN ? (nb_stats < 0 ? 0 : nb_stats < NB ? nb_stats : NB) : 0;
  __shared__ float s_red[(NB + 1) * 2 * 4];
  __shared__ float s_redm[SOUT ? NB * 4 : 1];
  __shared__ float s_red2[4];
  // sw (and sw_mlp) are shared by every row (cacheable)
  float4 swv[K3S_SLOTS][2], swm[SOUT ? K3S_SLOTS : 1][2];
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    swv[s][0] = *(const float4*)(sw + L.off(s));
    swv[s][1] = *(const float4*)(sw + L.off(s) + 4);
    if constexpr (SOUT) {
      swm[s][0] = *(const float4*)(sw_mlp + L.off(s));
      swm[s][1] = *(const float4*)(sw_mlp + L.off(s) + 4);
    }
  }

  // gamma is loaded with sw where the registers allow it (measured: the
  // statistics-writing push entries and nb above 6 lose occupancy), otherwise
  // at the normed stores
  constexpr bool GEARLY = !SOUT && NB <= 6;
  k3_u4 gv[K3S_SLOTS];
  if constexpr (GEARLY) {
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) gv[s] = k3_ld16(gamma + L.off(s));
  }
  pre(pv);
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    if (!L.valid(s)) continue;
    if (pvst.cached) k3_st16(pvst.cached + L.off(s), pv[s]);
    if (pvst.nt0) k3_st16_nt(pvst.nt0 + L.off(s), pv[s]);
    if (pvst.nt1) k3_st16_nt(pvst.nt1 + L.off(s), pv[s]);
  }
  // pass 1: sum x^2 and sum x * sw per candidate (prefix at index NB), chained
  // over the reference thread's steps by the hand-over
  float sq[NB + 1], dp[NB + 1], dm[SOUT ? NB : 1];
#pragma unroll
  for (int c = 0; c <= NB; ++c) { sq[c] = 0.0f; dp[c] = 0.0f; }
#pragma unroll
  for (int c = 0; c < (SOUT ? NB : 1); ++c) dm[c] = 0.0f;
  auto run = [&](int n) {
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) {
      if (s >= n) break;
      const float wv[8] = {swv[s][0].x, swv[s][0].y, swv[s][0].z, swv[s][0].w,
                           swv[s][1].x, swv[s][1].y, swv[s][1].z, swv[s][1].w};
      float mv[8];
      if constexpr (SOUT) {
        const float4 ma = swm[SOUT ? s : 0][0], mb = swm[SOUT ? s : 0][1];
        mv[0] = ma.x; mv[1] = ma.y; mv[2] = ma.z; mv[3] = ma.w;
        mv[4] = mb.x; mv[5] = mb.y; mv[6] = mb.z; mv[7] = mb.w;
      }
#pragma unroll
      for (int c = 0; c <= NB; ++c) {
        if (SIN && c < ns) continue;
        const k3_u4 x = c < NB ? xc[c < NB ? c : 0][s] : pv[s];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = k3_bf_lo(x[j]), hi = k3_bf_hi(x[j]);
          sq[c] = __builtin_fmaf(lo, lo, sq[c]);
          sq[c] = __builtin_fmaf(hi, hi, sq[c]);
          dp[c] = __builtin_fmaf(lo, wv[2 * j], dp[c]);
          dp[c] = __builtin_fmaf(hi, wv[2 * j + 1], dp[c]);
          if constexpr (SOUT) {
            if (c < NB) {
              dm[c < NB ? c : 0] = __builtin_fmaf(lo, mv[2 * j], dm[c < NB ? c : 0]);
              dm[c < NB ? c : 0] = __builtin_fmaf(hi, mv[2 * j + 1], dm[c < NB ? c : 0]);
            }
          }
        }
      }
      // slot by slot: the next slot is unpacked after this slot's chains
#pragma unroll
      for (int c = 0; c <= NB; ++c) asm volatile("" : "+v"(sq[c]), "+v"(dp[c]));
#pragma unroll
      for (int c = 0; c < (SOUT ? NB : 0); ++c) asm volatile("" : "+v"(dm[c]));
      if (s + 1 < n) {
#pragma unroll
        for (int c = 0; c < NB; ++c) asm volatile("" : "+v"(xc[c][s + 1 < K3S_SLOTS ? s + 1 : 0]));
        asm volatile("" : "+v"(pv[s + 1 < K3S_SLOTS ? s + 1 : 0]));
      }
    }
  };
  // Each use of a held row unpacks it again: the empty asm makes the packed
  // form the only live copy, so the unpacked floats of one run (twice the
  // registers) are not kept alive into the next run or pass 2.
  auto pin = [&]() {
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
      for (int s = 0; s < K3S_SLOTS; ++s) asm volatile("" : "+v"(xc[c][s]));
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) asm volatile("" : "+v"(pv[s]));
  };
  run(K3S_SLOTS);
#pragma unroll
  for (int c = 0; c <= NB; ++c) { sq[c] = k3s_handover(sq[c]); dp[c] = k3s_handover(dp[c]); }
#pragma unroll
  for (int c = 0; c < (SOUT ? NB : 0); ++c) dm[c] = k3s_handover(dm[c]);
  pin();
  run(K3_KVPT - K3S_SLOTS);
  pin();
#pragma unroll
  for (int c = 0; c <= NB; ++c) {
    if (SIN && c < ns) continue;
    const float s = k3_sum32(sq[c]);
    const float d = k3_sum32(dp[c]);
    if (L.lane == 32) { s_red[(2 * c) * 4 + L.w] = s; s_red[(2 * c + 1) * 4 + L.w] = d; }
    if constexpr (SOUT) {
      if (c < NB) {
        const float mm = k3_sum32(dm[c < NB ? c : 0]);
        if (L.lane == 32) s_redm[c * 4 + L.w] = mm;
      }
    }
  }
  __syncthreads();

  // scores and softmax (as the 128-thread body: lane c of each half-wave takes
  // candidate c; both halves compute the same values)
  const int lane32 = L.lane & 31;
  float sc = -3.0e38f;
  if (lane32 <= NB) {
    float sqv = 0.0f, dpv = 0.0f;
    if (SIN && lane32 < ns) {
      sqv = stats_in[2 * lane32];
      dpv = stats_in[2 * lane32 + 1];
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sqv += s_red[(2 * lane32) * 4 + w];
        dpv += s_red[(2 * lane32 + 1) * 4 + w];
      }
    }
    if constexpr (SOUT) {
      if (L.w == 0 && L.h == 0 && lane32 < NB) {
        float dmv = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) dmv += s_redm[lane32 * 4 + w];
        stats_out[2 * lane32] = sqv;
        stats_out[2 * lane32 + 1] = dmv;
      }
    }
    sc = dpv * k3_row_rscale(sqv, eps);
  }
  const float mx = k3_max32(sc);
  float ex = 0.0f;
  if (lane32 <= NB) {
    const float d = sc - mx;
    ex = d < -87.0f ? 0.0f : k3_expf(d);
  }
  const float den = k3_sum32(ex);
  const float pmine = ex / den;
  const int base = L.lane & 32;
  float p[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) p[c] = __shfl(pmine, base + c, 64);
  const float pp = __shfl(pmine, base + NB, 64);

  // pass 2: f32 mix of the lane's slots from registers, one bf16 landing per value
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = pp * k3_bf_lo(pv[s][j]);
      acc[2 * j + 1] = pp * k3_bf_hi(pv[s][j]);
    }
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = __builtin_fmaf(p[c], k3_bf_lo(xc[c][s][j]), acc[2 * j]);
        acc[2 * j + 1] = __builtin_fmaf(p[c], k3_bf_hi(xc[c][s][j]), acc[2 * j + 1]);
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) pv[s][j] = k3_pack_bf2(acc[2 * j], acc[2 * j + 1]);
    asm volatile("" : "+v"(pv[s]));
    if (s + 1 < K3S_SLOTS) {
#pragma unroll
      for (int c = 0; c < NB; ++c) asm volatile("" : "+v"(xc[c][s + 1 < K3S_SLOTS ? s + 1 : 0]));
    }
  }

  // RMS of the mixed row, normed = bf16(bf16(mixed * r) (x) gamma)
  const float r = k3_row_rscale(k3s_row_sumsq_total(pv, s_red2, L), eps);
  k3_u4 nv[K3S_SLOTS];
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) {
    const k3_u4 g = GEARLY ? gv[s] : k3_ld16(gamma + L.off(s));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      nv[s][j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(pv[s][j]) * r, k3_bf_hi(pv[s][j]) * r), g[j]);
    if (L.valid(s)) k3_st16_nt(dst.row + L.off(s), nv[s]);
  }
  if (dst.peer) {
#pragma unroll
    for (int q = 0; q < K3_MAX_RANKS; ++q) {
      if (q >= dst.nr) break;
      if (q == dst.rank) continue;
      uint16_t* prow = (uint16_t*)(uintptr_t)dst.peer[q] + dst.off;
#pragma unroll
      for (int s = 0; s < K3S_SLOTS; ++s)
        if (L.valid(s)) k3_st16_nt_g(prow + L.off(s), nv[s]);
    }
  }
}

// K1b entry body (landing add, then the row body) for a compile-time nb.
template <int NB, int MODE = 0>
K3_DEV void k3s_land_add_attnres_rms_body(const k3_land_t* __restrict__ partial,
                                          const uint16_t* __restrict__ prefix,
                                          const uint16_t* __restrict__ blocks,
                                          const float* __restrict__ sw,
                                          const uint16_t* __restrict__ gamma,
                                          uint16_t* __restrict__ prefix2,
                                          uint16_t* __restrict__ normed, int snapshot, int B,
                                          const float* __restrict__ stats = nullptr,
                                          int nb_stats = 0) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const K3sLane L = k3s_lane();
  const size_t row = (size_t)b * K3_H;
  // every load of the row (partial, prefix, the candidates) goes out before the
  // first store, which a later load's wait would otherwise include
  k3_u4 pv[K3S_SLOTS], pr[K3S_SLOTS];
#pragma unroll
  for (int s = 0; s < K3S_SLOTS; ++s) pv[s] = k3_load_land(partial, row + L.off(s));
  if (!snapshot) {
#pragma unroll
    for (int s = 0; s < K3S_SLOTS; ++s) pr[s] = k3_ld16_nt(prefix + row + L.off(s));
  }
  k3_u4 xc[NB][K3S_SLOTS];
  k3s_load_candidates<NB>(xc, blocks + (size_t)b * K3_NB_MAX * K3_H, L);
  const bool have_stats = MODE != 0 && stats != nullptr;
  const K3NormedDst dst = {normed + row, nullptr, 0, 0, 1};
  const K3sPvStores pvst = {nullptr, prefix2 + row, nullptr};
  auto land = [&](k3_u4* p) {
    if (!snapshot) {
#pragma unroll
      for (int s = 0; s < K3S_SLOTS; ++s) p[s] = k3_add_land(pr[s], p[s]);
    }
  };
  // From nb 2 the landing add runs after the body has issued its own loads (sw,
  // gamma), which then do not wait for the landing operands (B 4096, back to
  // back: nb 4 / 6 / 8 82.1 / 106.5 / 127.6 -> 80.9 / 103.1 / 124.9 us, identical
  // outputs); at nb 1 the extra live registers cost a wave per SIMD (93 -> 105)
  // and it measured 0.5-1.5% slower, so the add stays ahead there.
  const float* st = have_stats ? stats + (size_t)b * K3_NB_MAX * 2 : nullptr;
  const int ns = have_stats ? nb_stats : 0;
  if constexpr (NB == 1) {
    land(pv);
    k3s_attnres_rms_row<NB, MODE>(xc, pv, sw, gamma, dst, pvst, K3_EPS, L, st, ns);
  } else {
    k3s_attnres_rms_row<NB, MODE>(xc, pv, sw, gamma, dst, pvst, K3_EPS, L, st, ns, nullptr,
                                  nullptr, land);
  }
}
