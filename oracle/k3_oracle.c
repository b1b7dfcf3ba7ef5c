/* CPU oracle, part 1: numerics, K1 residual family, MXFP8, per-tensor fp8.
 * TEST INFRASTRUCTURE ONLY (see k3_oracle.h). */
#include "k3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define H 7168
#define NB_MAX 8
#define THREADS 128
#define KVPT 7

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int k3o_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Timing support for the CPU baseline: dst <- src split over the OpenMP threads in
 * 64 KB pieces, so that the pages of a freshly allocated dst are first touched by
 * the threads that later read them (first-touch NUMA placement). */
void k3o_par_copy(void* dst, const void* src, size_t n) {
  const long long chunks = (long long)((n + 65535) / 65536);
#pragma omp parallel for schedule(static)
  for (long long c = 0; c < chunks; ++c) {
    const size_t o = (size_t)c * 65536, m = n - o < 65536 ? n - o : 65536;
    memcpy((char*)dst + o, (const char*)src + o, m);
  }
}

/* ---------------------------------------------------------------- bf16 */
float k3o_bf2f(uint16_t h) { return bitsf((uint32_t)h << 16); }

/* IEEE round-to-nearest-even f32 -> bf16 (cuda_bf16 __float2bfloat16_rn
 * semantics).  NaN keeps its sign and is quieted. */
uint16_t k3o_f2bf(float f) {
  const uint32_t u = fbits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}
static inline float land(float f) { return k3o_bf2f(k3o_f2bf(f)); }

void k3o_f2bf_n(const float* x, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = k3o_f2bf(x[i]);
}

/* ---------------------------------------------------------------- e4m3 */
/* OCP FP8 E4M3 (no infinities; 0x7f / 0xff NaN; largest finite 448),
 * round to nearest even, saturating to +-448 (the __NV_SATFINITE mode used by
 * k3_moe_prefill_v4.cu:136 and k3_quant_fp8_pair_v2.cu:78-88).  Computed in
 * double, where every scaling below is exact. */
uint8_t k3o_e4m3(float x) {
  const uint8_t sign = (uint8_t)((fbits(x) >> 24) & 0x80u);
  if (isnan(x)) return 0x7f; /* canonical NaN of the saturating conversion */
  const double a = fabs((double)x);
  if (a >= 448.0) return (uint8_t)(sign | 0x7e);
  if (a < 0x1p-6) {                       /* subnormal quantum 2^-9 */
    const int r = (int)nearbyint(a * 512.0);
    return (uint8_t)(sign | (r >= 8 ? 0x08 : r));
  }
  int E;
  frexp(a, &E);                            /* a = f 2^E, f in [0.5, 1) */
  int e = E - 1;                           /* a in [2^e, 2^(e+1)) */
  int r = (int)nearbyint(ldexp(a, 3 - e)); /* significand in [8, 16] */
  if (r == 16) { r = 8; ++e; }
  if (e > 8 || (e == 8 && r > 14)) return (uint8_t)(sign | 0x7e);
  return (uint8_t)(sign | ((e + 7) << 3) | (r - 8));
}

float k3o_e4m3_decode(uint8_t c) {
  const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

void k3o_e4m3_n(const float* x, uint8_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = k3o_e4m3(x[i]);
}

/* ---------------------------------------------------------------- exp */
/* Deterministic exp: x = n ln2 + r (Cody-Waite, two-part ln2 whose high part
 * has 12 trailing zero bits), e^r by the degree-7 Taylor polynomial (Horner,
 * fmaf), scaled by 2^n.  Replaces CUDA expf / __expf (k3_router_argmax.cu:101,
 * k3_residual_v2.cu:183, k3_kda_out_gate_v3.cu:101).  Valid on [-87, 88.72]. */
float k3o_expf(float x) {
  const float n = rintf(x * 0x1.715476p+0f);
  float r = fmaf(n, -0x1.62e4p-1f, x);
  r = fmaf(n, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

void k3o_expf_n(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = k3o_expf(x[i]);
}

/* 1 / (1 + e^-x) (k3_router_argmax.cu:101 computes 1.0f / (1.0f + expf(-S))).
 * With t = -x: t at or above 0x1.62e430p+6 (88.7228...) makes the f32 e^t
 * overflow, so the quotient is 1 / (1 + inf) = 0; below -87, 1 + e^t rounds
 * to 1 exactly, so t is clamped there (keeps k3o_expf in its normal range).
 * NaN propagates. */
float k3o_sigmoid(float x) {
  const float t = -x;
  if (t >= 0x1.62e430p+6f) return 0.0f;
  return 1.0f / (1.0f + k3o_expf(t < -87.0f ? -87.0f : t));
}

/* ---------------------------------------------------------------- reductions */
/* xor butterfly over n (power of two) lanes: offsets n/2 .. 1; returns lane 0. */
static float bfly_sum(const float* v, int n) {
  float a[64], b[64];
  memcpy(a, v, sizeof(float) * (size_t)n);
  for (int o = n / 2; o > 0; o >>= 1) {
    for (int i = 0; i < n; ++i) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof(float) * (size_t)n);
  }
  return a[0];
}

/* Block total of 128 per-thread partials: butterfly per 32-lane warp, then the
 * four warp partials in warp order (k3_residual_v2.cu:235-242). */
static float block_sum128(const float* part) {
  float tot = 0.0f;
  for (int w = 0; w < 4; ++w) tot += bfly_sum(part + 32 * w, 32);
  return tot;
}

/* rsqrtf(sum * (1/H) + eps) of the reference, contracted to one fma; the
 * approximate rsqrtf is replaced by a correctly rounded 1 / sqrt. */
static inline float rscale(float tot, float eps) {
  return 1.0f / sqrtf(fmaf(tot, 1.0f / (float)H, eps));
}

/* ---------------------------------------------------------------- K1 row */
/* attnres_rms_row (k3_residual_v2.cu:107-257).  pv holds the prefix
 * candidate (bf16 values as f32) and is replaced by the mixed row; thread t
 * of 128 owns elements 8(t + 128 v) .. +8, v < 7. */
/* sw_mlp / stats_out: res_in's hand-off (k3_residual_push_stats.cu:176-263):
 * stats_out[c] = (sum x^2, sum x * sw_mlp) of block candidate c < nb, summed
 * in the same order as sq / dp.  stats_in / nb_stats: res_mlp's side
 * (k3_residual_nb_stats.cu:176-258): candidates c < min(nb_stats, nb) take
 * (sq, dp) from stats_in[c].  Both are [NB_MAX][2]. */
static void attnres_rms_row_ex(const uint16_t* blk_row, float* pv, const float* sw,
                               const uint16_t* gamma, uint16_t* normed_row, int nb, float eps,
                               const float* sw_mlp, float* stats_out, const float* stats_in,
                               int nb_stats) {
  const int ns = stats_in ? (nb_stats < 0 ? 0 : nb_stats < nb ? nb_stats : nb) : 0;
  if (nb > 0) {
    /* pass 1 (k3_residual_v2.cu:124-162): per-thread serial sums */
    float sq[NB_MAX + 1][THREADS], dp[NB_MAX + 1][THREADS], dm[NB_MAX][THREADS];
    for (int t = 0; t < THREADS; ++t) {
      float s[NB_MAX + 1] = {0}, d[NB_MAX + 1] = {0}, m[NB_MAX] = {0};
      for (int v = 0; v < KVPT; ++v) {
        const int u = (t + v * THREADS) * 8;
        for (int j = 0; j < 8; ++j) {
          const float f = pv[u + j];
          s[NB_MAX] = fmaf(f, f, s[NB_MAX]);
          d[NB_MAX] = fmaf(f, sw[u + j], d[NB_MAX]);
        }
        for (int c = ns; c < nb; ++c)
          for (int j = 0; j < 8; ++j) {
            const float f = k3o_bf2f(blk_row[(size_t)c * H + u + j]);
            s[c] = fmaf(f, f, s[c]);
            d[c] = fmaf(f, sw[u + j], d[c]);
            if (sw_mlp) m[c] = fmaf(f, sw_mlp[u + j], m[c]);
          }
      }
      for (int c = 0; c <= NB_MAX; ++c) { sq[c][t] = s[c]; dp[c][t] = d[c]; }
      for (int c = 0; c < NB_MAX; ++c) dm[c][t] = m[c];
    }
    /* candidate order: blocks 0..nb-1, then the prefix (k3_residual_v2.cu:154-161) */
    float sc[32], ex[32], p[NB_MAX + 1];
    const int ncand = nb + 1;
    float mx = -3.0e38f;
    for (int c = 0; c < ncand; ++c) {
      const int src = c < nb ? c : NB_MAX;
      float sqv = 0.0f, dpv = 0.0f;
      if (c < ns) {
        sqv = stats_in[2 * c];
        dpv = stats_in[2 * c + 1];
      } else {
        for (int w = 0; w < 4; ++w) {
          sqv += bfly_sum(&sq[src][32 * w], 32);
          dpv += bfly_sum(&dp[src][32 * w], 32);
        }
      }
      if (stats_out && c < nb) {
        float dmv = 0.0f;
        for (int w = 0; w < 4; ++w) dmv += bfly_sum(&dm[c][32 * w], 32);
        stats_out[2 * c] = sqv;
        stats_out[2 * c + 1] = dmv;
      }
      sc[c] = dpv * rscale(sqv, eps);
      mx = fmaxf(mx, sc[c]);
    }
    for (int c = 0; c < 32; ++c) {
      ex[c] = 0.0f;
      if (c < ncand) {
        const float d = sc[c] - mx;
        ex[c] = d < -87.0f ? 0.0f : k3o_expf(d); /* __expf(sc - mx), 183 */
      }
    }
    const float den = bfly_sum(ex, 32);
    for (int c = 0; c < ncand; ++c) p[c] = ex[c] / den;
    /* pass 2 (k3_residual_v2.cu:193-222): acc = p_prefix x + sum_c p_c x_c */
    for (int i = 0; i < H; ++i) {
      float acc = p[nb] * pv[i];
      for (int c = 0; c < nb; ++c) acc = fmaf(p[c], k3o_bf2f(blk_row[(size_t)c * H + i]), acc);
      pv[i] = land(acc);
    }
  }
  /* RMS (k3_residual_v2.cu:226-256) */
  float part[THREADS];
  for (int t = 0; t < THREADS; ++t) {
    float s = 0.0f;
    for (int v = 0; v < KVPT; ++v) {
      const int u = (t + v * THREADS) * 8;
      for (int j = 0; j < 8; ++j) s = fmaf(pv[u + j], pv[u + j], s);
    }
    part[t] = s;
  }
  const float r = rscale(block_sum128(part), eps);
  for (int i = 0; i < H; ++i) {
    const float y = land(pv[i] * r);
    normed_row[i] = k3o_f2bf(y * k3o_bf2f(gamma[i])); /* __hmul2: exact product, one RNE */
  }
}

static void attnres_rms_row(const uint16_t* blk_row, float* pv, const float* sw,
                            const uint16_t* gamma, uint16_t* normed_row, int nb, float eps) {
  attnres_rms_row_ex(blk_row, pv, sw, gamma, normed_row, nb, eps, NULL, NULL, NULL, 0);
}

/* K1b kern_k3_land_add_attnres_rms (k3_residual_v2.cu:295-345); with stats,
 * the res_mlp entries of k3_residual_nb_stats.cu:366-811 (stats [B, 8, 2]). */
void k3o_land_add_attnres_rms_stats(const uint16_t* partial_bf16, const float* partial_f32,
                                    const uint16_t* prefix, const uint16_t* blocks,
                                    const float* sw, const uint16_t* gamma, uint16_t* prefix2,
                                    uint16_t* normed, int nb, int snapshot, int B, float eps,
                                    const float* stats, int nb_stats) {
  if (nb < 0 || nb > NB_MAX) return;
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b) {
    float* pv = (float*)malloc(sizeof(float) * H);
    for (int i = 0; i < H; ++i) {
      const size_t o = (size_t)b * H + i;
      const float l = partial_bf16 ? k3o_bf2f(partial_bf16[o]) : land(partial_f32[o]);
      const float v = snapshot ? l : land(k3o_bf2f(prefix[o]) + l);
      prefix2[o] = k3o_f2bf(v);
      pv[i] = v;
    }
    attnres_rms_row_ex(blocks + (size_t)b * NB_MAX * H, pv, sw, gamma, normed + (size_t)b * H,
                       nb, eps, NULL, NULL, stats ? stats + (size_t)b * NB_MAX * 2 : NULL,
                       nb_stats);
    free(pv);
  }
}

void k3o_land_add_attnres_rms(const uint16_t* partial_bf16, const float* partial_f32,
                              const uint16_t* prefix, const uint16_t* blocks,
                              const float* sw, const uint16_t* gamma, uint16_t* prefix2,
                              uint16_t* normed, int nb, int snapshot, int B, float eps) {
  k3o_land_add_attnres_rms_stats(partial_bf16, partial_f32, prefix, blocks, sw, gamma, prefix2,
                                 normed, nb, snapshot, B, eps, NULL, 0);
}

/* K1a kern_k3_attnres_rms (k3_residual_v2.cu:260-284); with sw_mlp / stats,
 * res_in's statistics hand-off (k3_residual_push_stats.cu:354-385).  The push
 * entries (k3_residual_push_v3.cu:324-351) store this normed row into every
 * rank's normed_all; the checker computes the row once. */
void k3o_attnres_rms_stats(const uint16_t* prefix, uint16_t* blocks, const float* sw,
                           const uint16_t* gamma, uint16_t* normed, int nb, int snapshot, int B,
                           float eps, const float* sw_mlp, float* stats) {
  if (nb < 0 || nb > NB_MAX) return;
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b) {
    float* pv = (float*)malloc(sizeof(float) * H);
    for (int i = 0; i < H; ++i) pv[i] = k3o_bf2f(prefix[(size_t)b * H + i]);
    if (snapshot && nb < NB_MAX)
      memcpy(blocks + ((size_t)b * NB_MAX + nb) * H, prefix + (size_t)b * H, 2 * H);
    attnres_rms_row_ex(blocks + (size_t)b * NB_MAX * H, pv, sw, gamma, normed + (size_t)b * H, nb,
                       eps, stats ? sw_mlp : NULL, stats ? stats + (size_t)b * NB_MAX * 2 : NULL,
                       NULL, 0);
    free(pv);
  }
}

void k3o_attnres_rms(const uint16_t* prefix, uint16_t* blocks, const float* sw,
                     const uint16_t* gamma, uint16_t* normed, int nb, int snapshot, int B,
                     float eps) {
  k3o_attnres_rms_stats(prefix, blocks, sw, gamma, normed, nb, snapshot, B, eps, NULL, NULL);
}

/* kern_k3_land_add2_bf16 (k3_land_bf16.cu:84-140): K1c with bf16 partials,
 * hidden = bf16(f32(prefix2) + f32(p1) [+ f32(p2)]), left to right. */
void k3o_land_add2_bf16(const uint16_t* p1, const uint16_t* p2, const uint16_t* prefix2,
                        uint16_t* hidden, int two, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < H; ++i) {
      const size_t o = (size_t)b * H + i;
      float x = k3o_bf2f(prefix2[o]) + k3o_bf2f(p1[o]);
      if (two) x += k3o_bf2f(p2[o]);
      hidden[o] = k3o_f2bf(x);
    }
}

/* K1c kern_k3_land_add2 (k3_residual_v2.cu:349-392). */
void k3o_land_add2(const float* p1, const float* p2, const uint16_t* prefix2, uint16_t* hidden,
                   int two, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < H; ++i) {
      const size_t o = (size_t)b * H + i;
      float x = k3o_bf2f(prefix2[o]) + land(p1[o]);
      if (two) x += land(p2[o]);
      hidden[o] = k3o_f2bf(x);
    }
}

/* ---------------------------------------------------------------- MXFP8 */
/* e = amax > 0 ? clamp(ceil(log2(amax / 448)), -127, 127) : 0
 * (k3_moe_prefill_v4.cu:130).  log2 in double of the f32 quotient; an
 * infinite quotient saturates to 127 as the float->int conversion does. */
int k3o_mx_exp(float amax) {
  if (!(amax > 0.0f)) return 0;
  const float qt = amax / 448.0f;
  if (isinf(qt)) return 127;
  int e = (int)ceil(log2((double)qt));
  if (e < -127) e = -127;
  if (e > 127) e = 127;
  return e;
}

/* max(a, b) ignoring a NaN operand, signalling NaN included: the reference's
 * fmaxf (PTX max.f32) returns the other operand for any NaN, where glibc's
 * fmaxf follows IEEE 754-2008 maxNum and turns a signalling NaN (a bf16 NaN
 * pattern with bit 6 clear widens to one) into a quiet NaN result. */
static float max_nonan(float a, float b) {
  if (isnan(b)) return a;
  if (isnan(a)) return b;
  return b > a ? b : a;
}

static void mx_block(const float* v, uint8_t* q, uint8_t* sf) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = max_nonan(amax, fabsf(v[j]));
  const int e = k3o_mx_exp(amax);
  const float s = ldexpf(1.0f, -e); /* exp2f(-e): an exact power of two */
  *sf = (uint8_t)(e + 127);
  for (int j = 0; j < 32; ++j) q[j] = k3o_e4m3(v[j] * s);
}

/* kern_k3_moe_quant (k3_moe_prefill_v4.cu:111-140): blocks of 32 over the flat
 * element order. */
void k3o_moe_quant(const uint16_t* x, uint8_t* q, uint8_t* sf, int rows, int cols) {
  const long long nblk = (long long)rows * cols / 32;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < nblk; ++i) {
    float v[32];
    for (int j = 0; j < 32; ++j) v[j] = k3o_bf2f(x[i * 32 + j]);
    mx_block(v, q + i * 32, sf + i);
  }
}

/* Fused residual add + RMSNorm + MXFP8: K1b with nb = 0, snapshot = 0,
 * LAND_BF16 (k3_residual_v2.cu:295-345, row body 226-256) followed by the
 * moe_quant block rule on the normed row (k3_moe_prefill_v4.cu:111-140). */
void k3o_residual_rms_mxfp8(const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
                            uint16_t* residual_out, uint8_t* q, uint8_t* sf, uint16_t* normed,
                            int B, float eps) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b) {
    float* pv = (float*)malloc(sizeof(float) * H);
    uint16_t nrow[H];
    for (int i = 0; i < H; ++i) {
      const size_t o = (size_t)b * H + i;
      const float v = land(k3o_bf2f(residual[o]) + k3o_bf2f(x[o]));
      residual_out[o] = k3o_f2bf(v);
      pv[i] = v;
    }
    attnres_rms_row(NULL, pv, NULL, gamma, nrow, 0, eps);
    for (int k = 0; k < H / 32; ++k) {
      float v[32];
      for (int j = 0; j < 32; ++j) v[j] = k3o_bf2f(nrow[32 * k + j]);
      mx_block(v, q + (size_t)b * H + 32 * k, sf + (size_t)b * (H / 32) + k);
    }
    if (normed) memcpy(normed + (size_t)b * H, nrow, sizeof(nrow));
    free(pv);
  }
}

/* ---------------------------------------------------------------- fp8 pair */
/* kern_quant_fp8_amax[_v2] (k3_quant_fp8_pair.cu:18-30; _v2.cu:42-61):
 * partials[b] = max |x| over block b's grid-stride slice of a grid of
 * nb_grid blocks x 256 threads.  v1 strides over elements, v2 over 8-element
 * vectors (with the n % 8 tail folded into block 0); v2 takes the max of
 * |bf16| bit patterns, identical for non-NaN inputs. */
void k3o_quant_fp8_amax(const uint16_t* x, int n, float* partials, int nb_grid, int v2) {
  const long long stride = (long long)nb_grid * 256;
#pragma omp parallel for schedule(static)
  for (int b = 0; b < nb_grid; ++b) {
    if (!v2) {
      float m = 0.0f;
      for (int t = 0; t < 256; ++t)
        for (long long i = (long long)b * 256 + t; i < n; i += stride)
          m = max_nonan(m, fabsf(k3o_bf2f(x[i])));
      partials[b] = m;
    } else {
      uint32_t m = 0;
      const long long nv = n >> 3;
      for (int t = 0; t < 256; ++t)
        for (long long i = (long long)b * 256 + t; i < nv; i += stride)
          for (int j = 0; j < 8; ++j) {
            const uint32_t a = x[i * 8 + j] & 0x7fffu;
            if (a > m) m = a;
          }
      if (b == 0)
        for (int t = 0; t < (n & 7); ++t) {
          const uint32_t a = x[nv * 8 + t] & 0x7fffu;
          if (a > m) m = a;
        }
      partials[b] = k3o_bf2f((uint16_t)m);
    }
  }
}

/* kern_quant_fp8_apply[_v2] (k3_quant_fp8_pair.cu:32-51; _v2.cu:63-95):
 * amax = max(partials[0..nb)), scale = amax > 0 ? amax / 448 : 1,
 * y = e4m3_satfinite(f32(x) * (1 / scale)). */
void k3o_quant_fp8_apply(const uint16_t* x, uint8_t* y, int n, const float* partials, int nb,
                         float* scale_out) {
  float amax = 0.0f;
  for (int b = 0; b < nb; ++b) amax = max_nonan(amax, partials[b]);
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  if (scale_out) *scale_out = scale;
  const float inv = 1.0f / scale;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) y[i] = k3o_e4m3(k3o_bf2f(x[i]) * inv);
}
