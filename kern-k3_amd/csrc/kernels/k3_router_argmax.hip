// Module k3_router_argmax[+TOPK=n]: MoE router top-k and the two-stage f32 argmax.
//
//   kern_k3_router_topk(S, bias, rs, idx, wts, B)      grid (B), block 256
//   k3h_router_topk_pairs(S, bias, rs, idx, wts, B)    grid ceil(B / 8), block 256
//   kern_k3_argmax_f32_partial(logits, pmax, pidx, n)  grid (B, PARTS), block 1024
//   kern_k3_argmax_f32_final(pmax, pidx, out, parts)   grid (B), block 64
//
// Entry names, parameters and launch geometry are the reference module's
// (k3_router_argmax.cu:7-23, 87, 186, 227; manifest op router_topk,
// k3-tp4-prefill-16k.json:404788).  EXPERTS = 224; TOPK defaults to 16 (the
// manifest ABI) and is a define (TOPK=8 serves the 8-of-224 routing).
//
// Router, per row b (k3_router_argmax.cu:25-40, 87-152):
//   sig_e = 1 / (1 + e^-S[b,e]);  key_e = ord(sig_e + bias_e)   (ord: monotone f32->u32)
//   TOPK picks of the largest key, ties -> smallest e; a pick's key drops to 0
//   (below ord of every real number).
//   wts[t] = (sig_t / (sum_t sig_t + 1e-20)) * f32(rs[0]); the sum is the xor
//   butterfly over the TOPK pick lanes (offsets TOPK/2 .. 1).
// e^x is the deterministic k3_expf, so sig and therefore every key and index
// are reproduced bit for bit by the CPU checker.  One wave does the row:
// expert e = lane + 64 j lives in slot j of lane `lane`.  In the manifest
// geometry the other three waves of the 256-thread block have no work;
// k3h_router_topk_pairs (no reference counterpart, below) gives each half-wave
// a row.
#include "../common/k3_dev.h"

#define EXPERTS 224
#ifndef TOPK
#define TOPK 16
#endif
#define RSLOTS ((EXPERTS + 63) / 64)  // 4 slots per lane
static_assert(TOPK >= 1 && TOPK <= 32 && (TOPK & (TOPK - 1)) == 0, "TOPK: power of two <= 32");

// Largest value over the wave, on every lane (DPP steps fused with the max:
// quad swaps, half-row and row mirrors, then the row broadcasts 15 and 31).
K3_DEV uint32_t k3_router_wave_max(uint32_t v) {
  uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_1032, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_2301, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_HALF_MIRROR, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_MIRROR, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K3_DPP_ROW_BCAST15, 0xa, 0xf, false);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K3_DPP_ROW_BCAST31, 0xc, 0xf, false);
  v = v > o ? v : o;
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Row b on one full wave (expert e = lane + 64 j in slot j of lane `lane`).
K3_DEV void k3_router_row(const float* __restrict__ S, const float* __restrict__ bias,
                          const uint16_t* __restrict__ rs, int* __restrict__ idx,
                          float* __restrict__ wts, int b, int lane) {
  const float* row = S + (size_t)b * EXPERTS;

  // Every logit and bias of the lane is requested before the first is used (the
  // slots past the last expert read expert EXPERTS - 1 and are masked below), so
  // the row costs one memory round trip; the logistic is evaluated branch-free.
  float sv_[RSLOTS], bv_[RSLOTS];
#pragma unroll
  for (int j = 0; j < RSLOTS; ++j) {
    const int e = lane + 64 * j;
    const int ec = e < EXPERTS ? e : EXPERTS - 1;
    sv_[j] = row[ec];
    bv_[j] = bias[ec];
  }
  uint32_t key[RSLOTS];
  float sig[RSLOTS];
#pragma unroll
  for (int j = 0; j < RSLOTS; ++j) {
    const bool ok = lane + 64 * j < EXPERTS;
    sig[j] = ok ? k3_sigmoid_nb(sv_[j]) : 0.0f;
    key[j] = ok ? k3_ord_f32(sig[j] + bv_[j]) : 0u;
  }

  // Each lane keeps its four (key, slot) sorted, largest key first and ties to
  // the smaller slot, so a pick is a DPP wave max over the lanes' heads and one
  // ballot; the winner's head advances.  The smallest expert id among the keys
  // equal to the maximum is always some lane's head, so when several heads hold
  // it (rare) a second wave max over 255 - (64 slot + lane) of those lanes picks
  // it, as the reference's order does.  Lane r < TOPK notes pick r's lane and
  // slot; the sigmoids are fetched once after the picks.
  uint32_t hk[RSLOTS];
  int jj[RSLOTS];
#pragma unroll
  for (int j = 0; j < RSLOTS; ++j) { hk[j] = key[j]; jj[j] = j; }
  auto cswap = [&](int x, int y) {  // order positions x < y
    const bool sw = hk[x] < hk[y] || (hk[x] == hk[y] && jj[x] > jj[y]);
    const uint32_t kx = hk[x], ky = hk[y];
    const int jx = jj[x], jy = jj[y];
    hk[x] = sw ? ky : kx; hk[y] = sw ? kx : ky;
    jj[x] = sw ? jy : jx; jj[y] = sw ? jx : jy;
  };
  static_assert(RSLOTS == 4, "four slots per lane");
  cswap(0, 1); cswap(2, 3); cswap(0, 2); cswap(1, 3); cswap(1, 2);

  int my_lw = 0, my_jw = 0;
  for (int r = 0; r < TOPK; ++r) {
    const uint32_t m = k3_router_wave_max(hk[0]);
    const unsigned long long mk = __ballot(hk[0] == m);
    int lw;
    if (__builtin_popcountll(mk) == 1) {
      lw = __builtin_ctzll(mk);
    } else {
      const uint32_t cand = hk[0] == m ? 255u - (uint32_t)(64 * jj[0] + lane) : 0u;
      lw = (int)((255u - k3_router_wave_max(cand)) & 63u);
    }
    const int jw = __builtin_amdgcn_readlane(jj[0], lw);
    if (lane == lw) {
#pragma unroll
      for (int j = 0; j + 1 < RSLOTS; ++j) { hk[j] = hk[j + 1]; jj[j] = jj[j + 1]; }
      hk[RSLOTS - 1] = 0u;
    }
    if (lane == r) { my_lw = lw; my_jw = jw; }
  }
  // pick r's sigmoid: slot my_jw of lane my_lw
  float my_sig = 0.0f;
#pragma unroll
  for (int j = 0; j < RSLOTS; ++j) {
    const float t = __shfl(sig[j], my_lw, 64);
    my_sig = my_jw == j ? t : my_sig;
  }
  const int my_idx = 64 * my_jw + my_lw;

  // renormalise over the TOPK pick lanes: butterfly TOPK/2 .. 1, identical bits on every lane
  float den = my_sig;
#pragma unroll
  for (int o = TOPK / 2; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  if (lane < TOPK) {
    const float rsf = k3_bf(rs[0]);
    wts[(size_t)b * TOPK + lane] = (my_sig / (den + 1e-20f)) * rsf;
    idx[(size_t)b * TOPK + lane] = my_idx;
  }
}

// Manifest geometry: one row per 256-thread workgroup, wave 0 does it.
extern "C" __global__ void __launch_bounds__(256) kern_k3_router_topk(
    const float* __restrict__ S, const float* __restrict__ bias, const uint16_t* __restrict__ rs,
    int* __restrict__ idx, float* __restrict__ wts, int B) {
  const int b = blockIdx.x;
  if (b >= B || threadIdx.x >= 64) return;
  k3_router_row(S, bias, rs, idx, wts, b, threadIdx.x);
}


// ---------------------------------------------------------------- two rows per wave
// The same contract with one row per half-wave (k3h_router_topk_pairs, no
// reference counterpart): grid ceil(B / 8), block 256.  Expert e = s + 32 j
// (s = lane % 32, j < 7) lives in slot j of lane s of its half; each lane keeps
// its seven (key, slot) sorted (a 16-comparator network: largest key first, ties
// to the smaller slot, which is the smaller expert id), so a pick is a max over
// the half's heads and one ballot, and the two rows share every instruction of
// the pick loop.  When several heads of a half hold its maximum (rare) a second
// max over 255 - e picks the smallest expert id, as in k3_router_row.
#define PSLOTS (EXPERTS / 32)  // 7 slots per lane
static_assert(EXPERTS % 32 == 0, "whole slots per half-wave");

// Largest value over the lane's half-wave, on every lane of it: four DPP steps
// give each 16-lane row its maximum, then v_permlane16_swap exchanges the
// half's two rows (rows 2k and 2k + 1; with both operands the same value, the
// two results hold the lane's own row and the other row of its pair).
K3_DEV uint32_t k3_router_half_max(uint32_t v) {
  uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_1032, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_2301, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_HALF_MIRROR, 0xf, 0xf, true);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_MIRROR, 0xf, 0xf, true);
  v = v > o ? v : o;
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return r[0] > r[1] ? r[0] : r[1];
}

extern "C" __global__ void __launch_bounds__(256) k3h_router_topk_pairs(
    const float* __restrict__ S, const float* __restrict__ bias, const uint16_t* __restrict__ rs,
    int* __restrict__ idx, float* __restrict__ wts, int B) {
  const int lane = threadIdx.x & 63, s = lane & 31, h = lane >> 5;
  const int b0 = 2 * (int)(blockIdx.x * 4 + (threadIdx.x >> 6));  // the wave's first row
  if (b0 >= B) return;                                              // whole wave
  const int b = b0 + h;
  const bool live = b < B;  // the second half of the last wave may have no row
  const float* row = S + (size_t)(live ? b : B - 1) * EXPERTS;

  float sv_[PSLOTS], bv_[PSLOTS];
#pragma unroll
  for (int j = 0; j < PSLOTS; ++j) {
    sv_[j] = row[s + 32 * j];
    bv_[j] = bias[s + 32 * j];
  }
  float sig[PSLOTS];
  uint32_t hk[PSLOTS];
  int jj[PSLOTS];
#pragma unroll
  for (int j = 0; j < PSLOTS; ++j) {
    sig[j] = k3_sigmoid_nb(sv_[j]);
    hk[j] = k3_ord_f32(sig[j] + bv_[j]);
    jj[j] = j;
  }
  auto cswap = [&](int x, int y) {  // order positions x < y (no short circuit: one select each)
    const bool sw = (hk[x] < hk[y]) | ((hk[x] == hk[y]) & (jj[x] > jj[y]));
    const uint32_t kx = hk[x], ky = hk[y];
    const int jx = jj[x], jy = jj[y];
    hk[x] = sw ? ky : kx; hk[y] = sw ? kx : ky;
    jj[x] = sw ? jy : jx; jj[y] = sw ? jx : jy;
  };
  static_assert(PSLOTS == 7, "the network sorts seven slots");
  cswap(0, 6); cswap(2, 3); cswap(4, 5);
  cswap(0, 2); cswap(1, 4); cswap(3, 6);
  cswap(0, 1); cswap(2, 5); cswap(3, 4);
  cswap(1, 2); cswap(4, 6);
  cswap(2, 3); cswap(4, 5);
  cswap(1, 2); cswap(3, 4); cswap(5, 6);

  int my_lw = 0, my_jw = 0;
  for (int r = 0; r < TOPK; ++r) {
    const uint32_t m = k3_router_half_max(hk[0]);
    const unsigned long long mk = __ballot(hk[0] == m);
    const uint32_t m0 = (uint32_t)mk, m1 = (uint32_t)(mk >> 32);
    int lw0, lw1;
    if (__builtin_popcount(m0) == 1 && __builtin_popcount(m1) == 1) {
      lw0 = __builtin_ctz(m0);
      lw1 = __builtin_ctz(m1);
    } else {
      const uint32_t cand = hk[0] == m ? 255u - (uint32_t)(32 * jj[0] + s) : 0u;
      const uint32_t cm = k3_router_half_max(cand);
      lw0 = (int)((255u - (uint32_t)__builtin_amdgcn_readlane((int)cm, 0)) & 31u);
      lw1 = (int)((255u - (uint32_t)__builtin_amdgcn_readlane((int)cm, 32)) & 31u);
    }
    const int jw0 = __builtin_amdgcn_readlane(jj[0], lw0);
    const int jw1 = __builtin_amdgcn_readlane(jj[0], 32 + lw1);
    const int lw = h ? lw1 : lw0, jw = h ? jw1 : jw0;
    if (s == lw) {
#pragma unroll
      for (int j = 0; j + 1 < PSLOTS; ++j) { hk[j] = hk[j + 1]; jj[j] = jj[j + 1]; }
      hk[PSLOTS - 1] = 0u;
    }
    if (s == r) { my_lw = lw; my_jw = jw; }
  }
  // pick r's sigmoid: slot my_jw of lane 32 h + my_lw
  float my_sig = 0.0f;
#pragma unroll
  for (int j = 0; j < PSLOTS; ++j) {
    const float t = __shfl(sig[j], 32 * h + my_lw, 64);
    my_sig = my_jw == j ? t : my_sig;
  }
  const int my_idx = 32 * my_jw + my_lw;
  // renormalise over the TOPK pick lanes of the half: the butterfly of k3_router_row
  float den = my_sig;
#pragma unroll
  for (int o = TOPK / 2; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  if (live && s < TOPK) {
    const float rsf = k3_bf(rs[0]);
    wts[(size_t)b * TOPK + s] = (my_sig / (den + 1e-20f)) * rsf;
    idx[(size_t)b * TOPK + s] = my_idx;
  }
}

// ---------------------------------------------------------------- argmax
#define ARGMAX_IDX_TOP 0x7fffffff

K3_DEV uint64_t k3_amax_key(float v, int i) {
  return ((uint64_t)k3_ord_f32(v) << 32) | (uint32_t)(ARGMAX_IDX_TOP - i);
}
K3_DEV float k3_unord_f32(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
K3_DEV uint64_t k3_wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
    const uint64_t p = ((uint64_t)hi << 32) | lo;
    v = v > p ? v : p;
  }
  return v;
}

// Stage 1 (k3_router_argmax.cu:186-225): row blockIdx.x, chunk blockIdx.y of
// ceil(n / PARTS) elements; best = max over the chunk of (ord(v), TOP - i):
// largest value, ties to the smallest index.  An empty chunk writes (-inf, TOP).
extern "C" __global__ void __launch_bounds__(1024) kern_k3_argmax_f32_partial(
    const float* __restrict__ logits, float* __restrict__ pmax, int* __restrict__ pidx, int n) {
  __shared__ uint64_t sm[16];
  const int parts = gridDim.y;
  const int chunk = (n + parts - 1) / parts;
  const int lo = blockIdx.y * chunk;
  const int hi = min(lo + chunk, n);
  const float* __restrict__ row = logits + (size_t)blockIdx.x * n;
  uint64_t best = 0ull;
  for (int j = lo + (int)threadIdx.x; j < hi; j += 1024) {
    const uint64_t k = k3_amax_key(row[j], j);
    best = best > k ? best : k;
  }
  best = k3_wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w) best = best > sm[w] ? best : sm[w];
    const int o = blockIdx.x * parts + blockIdx.y;
    if (best == 0ull) {
      pmax[o] = -__builtin_inff();
      pidx[o] = ARGMAX_IDX_TOP;
    } else {
      pmax[o] = k3_unord_f32((uint32_t)(best >> 32));
      pidx[o] = ARGMAX_IDX_TOP - (int)(uint32_t)(best & 0xffffffffull);
    }
  }
}

// Stage 2 (k3_router_argmax.cu:227-243): the same rule over the row's partials;
// out = the i64 index, or 0 when every chunk was empty.
extern "C" __global__ void __launch_bounds__(64) kern_k3_argmax_f32_final(
    const float* __restrict__ pmax, const int* __restrict__ pidx, long long* __restrict__ out,
    int parts) {
  const long long base = (long long)blockIdx.x * parts;
  uint64_t best = 0ull;
  for (int t = threadIdx.x; t < parts; t += 64) {
    const int i = pidx[base + t];
    if (i != ARGMAX_IDX_TOP) {
      const uint64_t k = k3_amax_key(pmax[base + t], i);
      best = best > k ? best : k;
    }
  }
  best = k3_wave_max_u64(best);
  if (threadIdx.x == 0)
    out[blockIdx.x] = best == 0ull ? 0ll : (long long)(ARGMAX_IDX_TOP - (int)(uint32_t)(best & 0xffffffffull));
}
