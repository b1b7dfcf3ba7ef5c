/* CPU oracle, part 2: MoE router top-k, argmax, EP routing tables, permute and
 * finalize.  TEST INFRASTRUCTURE ONLY (see k3_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "k3_oracle.h"

#define EXPERTS 224

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* monotone f32 -> u32 (k3_router_argmax.cu:70-76) */
uint32_t k3o_ord_f32(float f) {
  const uint32_t b = fbits(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static float unord_f32(uint32_t o) { return bitsf((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o); }

/* kern_k3_router_topk (k3_router_argmax.cu:87-152): sig = 1/(1+e^-S) (expf
 * replaced by the deterministic k3o_expf through k3o_sigmoid), key =
 * ord(sig + bias), topk sequential picks of the largest key with ties to the
 * smallest expert, a pick's key set to 0; wts = (sig / (butterfly sum + 1e-20))
 * * f32(rs). */
void k3o_router_topk(const float* S, const float* bias, const uint16_t* rs, int* idx, float* wts,
                     int B, int topk) {
  const float rsf = k3o_bf2f(rs[0]);
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b) {
    float sig[EXPERTS];
    uint32_t key[EXPERTS];
    for (int e = 0; e < EXPERTS; ++e) {
      sig[e] = k3o_sigmoid(S[(size_t)b * EXPERTS + e]);
      key[e] = k3o_ord_f32(sig[e] + bias[e]);
    }
    float ps[32] = {0};
    for (int r = 0; r < topk; ++r) {
      int best = 0;
      for (int e = 1; e < EXPERTS; ++e)
        if (key[e] > key[best]) best = e; /* strict: ties keep the smaller e */
      idx[(size_t)b * topk + r] = best;
      ps[r] = sig[best];
      key[best] = 0u;
    }
    /* xor butterfly over the topk lanes (offsets topk/2 .. 1) */
    float a[32], c[32];
    memcpy(a, ps, sizeof(a));
    for (int o = topk / 2; o > 0; o >>= 1) {
      for (int i = 0; i < topk; ++i) c[i] = a[i] + a[i ^ o];
      memcpy(a, c, sizeof(float) * (size_t)topk);
    }
    const float den = a[0];
    for (int r = 0; r < topk; ++r) wts[(size_t)b * topk + r] = (ps[r] / (den + 1e-20f)) * rsf;
  }
}

void k3o_sigmoid_n(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = k3o_sigmoid(x[i]);
}

/* kern_k3_argmax_f32_partial (k3_router_argmax.cu:186-225): best (value,
 * smallest index) per chunk of ceil(n / parts); empty chunk -> (-inf, TOP). */
#define ARGMAX_TOP 0x7fffffff
static uint64_t amax_key(float v, int i) {
  return ((uint64_t)k3o_ord_f32(v) << 32) | (uint32_t)(ARGMAX_TOP - i);
}
void k3o_argmax_partial(const float* logits, float* pmax, int* pidx, int B, int n, int parts) {
  const int chunk = (n + parts - 1) / parts;
  for (int b = 0; b < B; ++b)
    for (int y = 0; y < parts; ++y) {
      const int lo = y * chunk, hi = lo + chunk < n ? lo + chunk : n;
      uint64_t best = 0;
      for (int j = lo; j < hi; ++j) {
        const uint64_t k = amax_key(logits[(size_t)b * n + j], j);
        if (k > best) best = k;
      }
      const int o = b * parts + y;
      if (!best) { pmax[o] = -INFINITY; pidx[o] = ARGMAX_TOP; }
      else { pmax[o] = unord_f32((uint32_t)(best >> 32)); pidx[o] = ARGMAX_TOP - (int)(uint32_t)best; }
    }
}

/* kern_k3_argmax_f32_final (k3_router_argmax.cu:227-243). */
void k3o_argmax_final(const float* pmax, const int* pidx, long long* out, int B, int parts) {
  for (int b = 0; b < B; ++b) {
    uint64_t best = 0;
    for (int t = 0; t < parts; ++t) {
      const int i = pidx[(size_t)b * parts + t];
      if (i != ARGMAX_TOP) {
        const uint64_t k = amax_key(pmax[(size_t)b * parts + t], i);
        if (k > best) best = k;
      }
    }
    out[b] = best ? (long long)(ARGMAX_TOP - (int)(uint32_t)best) : 0;
  }
}

/* ---------------------------------------------------------------- EP routing */
/* local_expert (k3_moe_prefill_v4.cu:100-109): strided placement (id % ranks
 * == rank -> id / ranks) or block placement (id - rank E); -1 when another rank
 * owns the expert. */
int k3o_local_expert(int id, int rank, int E, int ep_ranks, int strided) {
  if (strided) {
    if (id % ep_ranks != rank) return -1;
    const int e = id / ep_ranks;
    return e < E ? e : -1;
  }
  const int e = id - rank * E;
  return (e >= 0 && e < E) ? e : -1;
}

/* kern_k3_moe_route_count (k3_moe_prefill_v4.cu:142-157): blockcount[b][e] =
 * the local expert e's ids among tokens [256 b, 256 b + 256). */
void k3o_route_count(const int* ids, int T, int topk, int rank, int E, int ep_ranks, int strided,
                     int* blockcount) {
  const int nblk = (T + 255) / 256;
  memset(blockcount, 0, sizeof(int) * (size_t)nblk * E);
  for (int t = 0; t < T; ++t)
    for (int k = 0; k < topk; ++k) {
      const int e = k3o_local_expert(ids[(size_t)t * topk + k], rank, E, ep_ranks, strided);
      if (e >= 0) ++blockcount[(t / 256) * E + e];
    }
}

/* kern_k3_moe_route_tables (k3_moe_prefill_v4.cu:159-203): expert offsets in
 * tile units (exclusive scan of ceil(count / tile)), per-(block, expert) first
 * rows, CTA tables, padding rows of each expert's last tile routed to token 0. */
void k3o_route_tables(const int* blockcount, int blocks, int E, int tile, int* blockoff,
                      int* cta_batch, int* cta_limit, int* num_non_exiting, int* total_padded,
                      int* route_map) {
  int count[64], off[65];
  for (int e = 0; e < E; ++e) {
    int run = 0;
    for (int b = 0; b < blocks; ++b) run += blockcount[b * E + e];
    count[e] = run;
  }
  int run = 0;
  for (int e = 0; e < E; ++e) { off[e] = run; run += (count[e] + tile - 1) / tile; }
  off[E] = run;
  *num_non_exiting = run;
  *total_padded = run * tile;
  for (int e = 0; e < E; ++e) {
    int r = off[e] * tile;
    for (int b = 0; b < blocks; ++b) { blockoff[b * E + e] = r; r += blockcount[b * E + e]; }
    for (int p = off[e] * tile + count[e]; p < off[e + 1] * tile; ++p) route_map[p] = 0;
  }
  for (int i = 0; i < off[E]; ++i) {
    int j = 0;
    while (off[j + 1] <= i) ++j;
    cta_batch[i] = j;
    const int lim = off[j] * tile + count[j];
    cta_limit[i] = (i + 1) * tile < lim ? (i + 1) * tile : lim;
  }
}

/* kern_k3_moe_route_scatter (k3_moe_prefill_v4.cu:205-252): the permuted row of
 * expanded id idx = t topk + k is blockoff[b][e] plus its rank among the
 * block's ids of expert e in ascending idx order (a stable counting sort);
 * route_map[row] = t, exp2perm[idx] = row or -1 when the expert is not local. */
void k3o_route_scatter(const int* ids, const int* blockoff, int T, int topk, int rank, int E,
                       int ep_ranks, int strided, int* route_map, int* exp2perm) {
  const int nblk = (T + 255) / 256;
  for (int b = 0; b < nblk; ++b) {
    int seen[64] = {0};
    const long long lo = (long long)b * 256 * topk;
    long long hi = lo + 256LL * topk;
    if (hi > (long long)T * topk) hi = (long long)T * topk;
    for (long long idx = lo; idx < hi; ++idx) {
      const int e = k3o_local_expert(ids[idx], rank, E, ep_ranks, strided);
      if (e < 0) { exp2perm[idx] = -1; continue; }
      const int row = blockoff[b * E + e] + seen[e]++;
      route_map[row] = (int)(idx / topk);
      exp2perm[idx] = row;
    }
  }
}

/* MXFP8 permute (new op; the reference gathers the same rows inside moe_fc1
 * through route_map, k3_moe_prefill_v4.cu:21-25): pq[r] = q[route_map[r]],
 * psf[r] = sf[route_map[r]] for r < total_padded. */
void k3o_moe_permute_mx(const uint8_t* q, const uint8_t* sf, const int* route_map,
                        int total_padded, int cols, uint8_t* pq, uint8_t* psf) {
  const int sfc = cols / 32;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < total_padded; ++r) {
    const int t = route_map[r];
    memcpy(pq + (size_t)r * cols, q + (size_t)t * cols, (size_t)cols);
    memcpy(psf + (size_t)r * sfc, sf + (size_t)t * sfc, (size_t)sfc);
  }
}

/* kern_k3_moe_finalize (k3_moe_prefill_v4.cu:254-302): out[t, c] = bf16(sum over
 * k ascending with exp2perm >= 0 of wts[t][k] * f32(fc2[row, c])), f32 accumulator
 * from 0 with one fma per term. */
void k3o_moe_finalize(const uint16_t* fc2, const int* exp2perm, const float* wts, uint16_t* out,
                      int T, int topk, int cols) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    int rows[32];
    float w[32];
    int n = 0;
    for (int k = 0; k < topk; ++k) {
      const int p = exp2perm[(size_t)t * topk + k];
      if (p >= 0) { rows[n] = p; w[n] = wts[(size_t)t * topk + k]; ++n; }
    }
    for (int c = 0; c < cols; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < n; ++i) acc = fmaf(w[i], k3o_bf2f(fc2[(size_t)rows[i] * cols + c]), acc);
      out[(size_t)t * cols + c] = k3o_f2bf(acc);
    }
  }
}

/* kern_k3_moe_w_shuffle / kern_k3_moe_sf_shuffle (k3_moe_prefill_v4.cu:304-327):
 * load-time layouts.  Row r of an expert's destination takes source row
 * shuffle(r) = (r/32)*32 + (r%8)*4 + (r%32)/8, after the gated interleave
 * (u odd -> n/2 + u/2, even -> u/2) when gated; the scales are re-laid in
 * 128x4 blocks. */
static int w_shuffle_row(int r, int n, int gated) {
  const int u = (r / 32) * 32 + (r % 8) * 4 + (r % 32) / 8;
  return gated ? (u % 2 ? n / 2 : 0) + u / 2 : u;
}
void k3o_moe_w_shuffle(const uint8_t* src, uint8_t* dst, int experts, int n, int row_bytes,
                       int gated) {
  for (int e = 0; e < experts; ++e)
    for (int r = 0; r < n; ++r)
      memcpy(dst + ((size_t)e * n + r) * row_bytes,
             src + ((size_t)e * n + w_shuffle_row(r, n, gated)) * row_bytes, (size_t)row_bytes);
}
void k3o_moe_sf_shuffle(const uint8_t* src, uint8_t* dst, int experts, int n, int kg, int gated) {
  for (int e = 0; e < experts; ++e)
    for (int r = 0; r < n; ++r)
      for (int c = 0; c < kg; ++c) {
        const long long at = ((long long)(r / 128) * (kg / 4) + c / 4) * 512 + (r % 32) * 16 +
                             ((r % 128) / 32) * 4 + c % 4;
        dst[(size_t)e * n * kg + at] = src[((size_t)e * n + w_shuffle_row(r, n, gated)) * kg + c];
      }
}
