// Module k3_router_argmax[+TOPK=n]: MoE router top-k and the two-stage f32 argmax.
//
//   kern_k3_router_topk(S, bias, rs, idx, wts, B)      grid (B), block 256
//   k3h_router_topk_rows(S, bias, rs, idx, wts, B)     grid ceil(B / 4), block 256
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
// k3h_router_topk_rows (no reference counterpart) gives each wave a row.
#include "../common/k3_dev.h"

#define EXPERTS 224
#ifndef TOPK
#define TOPK 16
#endif
#define RSLOTS ((EXPERTS + 63) / 64)  // 4 slots per lane
static_assert(TOPK >= 1 && TOPK <= 32 && (TOPK & (TOPK - 1)) == 0, "TOPK: power of two <= 32");

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

  // A pick is a DPP wave max of the keys (uniform) and a ballot per slot for the
  // lanes holding it: slots are scanned from the top so the lowest slot, and in
  // it the lowest lane, i.e. the smallest expert id, wins.  (Keeping a per-lane
  // best and breaking cross-lane ties by a second wave min only when a ballot
  // has more than one lane measured no faster: 16.0 against 15.8 us.)
  int my_idx = 0;
  float my_sig = 0.0f;
  for (int r = 0; r < TOPK; ++r) {
    uint32_t m = key[0];
#pragma unroll
    for (int j = 1; j < RSLOTS; ++j) m = m > key[j] ? m : key[j];
    m = k3_wave_max_u32_uniform(m);
    int jw = 0, lw = 0;
#pragma unroll
    for (int j = RSLOTS - 1; j >= 0; --j) {
      const unsigned long long mk = __ballot(key[j] == m);
      if (mk) { jw = j; lw = __builtin_ctzll(mk); }
    }
    float sv = sig[0];
#pragma unroll
    for (int j = 1; j < RSLOTS; ++j) sv = jw == j ? sig[j] : sv;
    const float sw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), lw));
#pragma unroll
    for (int j = 0; j < RSLOTS; ++j)
      if (j == jw && lane == lw) key[j] = 0u;
    if (lane == r) { my_idx = 64 * jw + lw; my_sig = sw; }
  }

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

// Same contract, one row per wave: grid ceil(B / 4), block 256.
extern "C" __global__ void __launch_bounds__(256) k3h_router_topk_rows(
    const float* __restrict__ S, const float* __restrict__ bias, const uint16_t* __restrict__ rs,
    int* __restrict__ idx, float* __restrict__ wts, int B) {
  const int b = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (b >= B) return;
  k3_router_row(S, bias, rs, idx, wts, b, threadIdx.x & 63);
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
