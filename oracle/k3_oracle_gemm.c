/* MoE expert GEMMs: the MX-scaled products that replace the reference's
 * prebuilt batched GEMMs moe_fc1 / moe_fc2 (manifest ops
 * k3-tp4-prefill-16k.json:405185 / 405419: MxE4m3 activations x MxE2m1 weights,
 * f32 accumulation, siTuGlu epilogue with per-expert alpha / beta that the
 * manifest fills with 4.0 and 25.0).  The reference kernels are binary-only and
 * absent, so this restates the mathematics of an MX block-scaled product
 * (OCP MX: value = element * 2^(E8M0 - 127), blocks of 32 along K) in double.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.py). */
#include "k3_oracle.h"

#include <math.h>
#include <stdlib.h>

/* OCP FP4 E2M1: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0; the
 * eight magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6. */
float k3o_e2m1_decode(uint8_t nib) {
  const int s = (nib >> 3) & 1, e = (nib >> 1) & 3, m = nib & 1;
  const float v = e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1);
  return s ? -v : v;
}

static float e8m0(uint8_t s) { return ldexpf(1.0f, (int)s - 127); }

/* out[r, n] (double) = sum_k a(src(r), k) w_e(n, k) for rows r of the route
 * tiles t < num_tiles whose expert e = cta_batch[t] is in [0, E); rows of other
 * tiles are left untouched.  a e4m3 [*, K] with a_sf [*, K/32]; w e2m1
 * [E, N, K/2] (low nibble = even k) with w_sf [E, N, K/32]; src(r) = a_rows[r]
 * (negative -> 0) or r. */
void k3o_moe_gemm_mx(const uint8_t* a, const uint8_t* a_sf, const int* a_rows, const uint8_t* w,
                     const uint8_t* w_sf, int num_tiles, const int* cta_batch, int E, int N, int K,
                     double* out) {
  const int KG = K / 32;
  float* wd = (float*)malloc(sizeof(float) * (size_t)N * K);
  for (int e = 0; e < E; ++e) {
    int used = 0;
    for (int t = 0; t < num_tiles; ++t) used |= cta_batch[t] == e;
    if (!used) continue;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint8_t* wr = w + ((size_t)e * N + n) * (K / 2);
      const uint8_t* sr = w_sf + ((size_t)e * N + n) * KG;
      for (int k = 0; k < K; ++k) {
        const uint8_t nib = (k & 1) ? (wr[k / 2] >> 4) : (wr[k / 2] & 15);
        wd[(size_t)n * K + k] = k3o_e2m1_decode(nib) * e8m0(sr[k / 32]);
      }
    }
    for (int t = 0; t < num_tiles; ++t) {
      if (cta_batch[t] != e) continue;
#pragma omp parallel for schedule(static)
      for (int i = 0; i < 128; ++i) {
        const int r = t * 128 + i;
        int src = a_rows ? a_rows[r] : r;
        if (src < 0) src = 0;
        double ad[8192];
        for (int k = 0; k < K; ++k)
          ad[k] = (double)k3o_e4m3_decode(a[(size_t)src * K + k]) *
                  (double)e8m0(a_sf[(size_t)src * KG + k / 32]);
        for (int n = 0; n < N; ++n) {
          const float* wn = wd + (size_t)n * K;
          double acc = 0.0;
          for (int k = 0; k < K; ++k) acc += ad[k] * (double)wn[k];
          out[(size_t)r * N + n] = acc;
        }
      }
    }
  }
  free(wd);
}

/* sum_k |a(src(r), k) w_e(n, k)|: the magnitude the accumulation error of a
 * reordered / reduced-precision sum is measured against. */
void k3o_moe_gemm_mx_abs(const uint8_t* a, const uint8_t* a_sf, const int* a_rows,
                         const uint8_t* w, const uint8_t* w_sf, int num_tiles,
                         const int* cta_batch, int E, int N, int K, double* out) {
  const int KG = K / 32;
  float* wd = (float*)malloc(sizeof(float) * (size_t)N * K);
  for (int e = 0; e < E; ++e) {
    int used = 0;
    for (int t = 0; t < num_tiles; ++t) used |= cta_batch[t] == e;
    if (!used) continue;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
      for (int k = 0; k < K; ++k) {
        const uint8_t* wr = w + ((size_t)e * N + n) * (K / 2);
        const uint8_t nib = (k & 1) ? (wr[k / 2] >> 4) : (wr[k / 2] & 15);
        wd[(size_t)n * K + k] =
            fabsf(k3o_e2m1_decode(nib) * e8m0(w_sf[((size_t)e * N + n) * KG + k / 32]));
      }
    for (int t = 0; t < num_tiles; ++t) {
      if (cta_batch[t] != e) continue;
#pragma omp parallel for schedule(static)
      for (int i = 0; i < 128; ++i) {
        const int r = t * 128 + i;
        int src = a_rows ? a_rows[r] : r;
        if (src < 0) src = 0;
        double ad[8192];
        for (int k = 0; k < K; ++k)
          ad[k] = fabs((double)k3o_e4m3_decode(a[(size_t)src * K + k]) *
                       (double)e8m0(a_sf[(size_t)src * KG + k / 32]));
        for (int n = 0; n < N; ++n) {
          double acc = 0.0;
          for (int k = 0; k < K; ++k) acc += ad[k] * (double)wd[(size_t)n * K + k];
          out[(size_t)r * N + n] = acc;
        }
      }
    }
  }
  free(wd);
}

/* The gated activation of the fc1 epilogue for general alpha / beta on
 * bf16-landed operands, exactly (double), returned as the f32 value that lands:
 * (alpha tanh(g / alpha) sigmoid(g)) (beta tanh(u * (1/beta))), with
 * u * (1/beta) the f32 product of u and the f32 reciprocal (for beta = 25 that
 * is the reference landing's u * 0.04f, so alpha = 4, beta = 25 gives k3o_situ). */
void k3o_situ_ab_n(const float* g, const float* u, float* y, size_t n, float alpha, float beta) {
  const float ib = 1.0f / beta;
  for (size_t i = 0; i < n; ++i) {
    const float uy = u[i] * ib;
    const double gate =
        (double)alpha * tanh((double)g[i] / (double)alpha) * (1.0 / (1.0 + exp(-(double)g[i])));
    const double up = (double)beta * tanh((double)uy);
    y[i] = (float)(gate * up);
  }
}
