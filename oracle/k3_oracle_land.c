/* CPU oracle, part 5: landing kernels of the shared-expert MLP and the MoE
 * latent norm (k3_land.cu, k3_land_bf16.cu, k3_situ_bf16.cu, k3_land_fused.cu).
 * TEST INFRASTRUCTURE ONLY (see k3_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "k3_oracle.h"

#define RMS_EPS 1e-5f

static inline float land(float f) { return k3o_bf2f(k3o_f2bf(f)); }

/* xor butterfly over 32 lanes (offsets 16 .. 1); the lane-0 value. */
static float bfly32(const float* v) {
  float a[32], b[32];
  memcpy(a, v, sizeof(a));
  for (int o = 16; o > 0; o >>= 1) {
    for (int i = 0; i < 32; ++i) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof(a));
  }
  return a[0];
}

/* block_sum of k3_land.cu:86-102 over nt threads' partials: a butterfly per
 * warp of 32, then warp 0 butterflies the nt/32 warp partials (zeros above). */
static float block_sum(const float* part, int nt) {
  float w[32] = {0};
  for (int k = 0; k < nt / 32; ++k) w[k] = bfly32(part + 32 * k);
  return bfly32(w);
}

/* One rms row with the reference's thread layout: nt threads; vector path
 * (h % 8 == 0) thread tid sums its vectors u = tid + nt r, u < nvec_max
 * (8 fma steps each); scalar path its elements i = tid + nt r.  The output is
 * bf16(x * r) (x) gamma, r = rsqrtf(sum / h + 1e-5) as 1 / sqrt (k3_land.cu:104-165,
 * k3_land_fused.cu:160-187).  Vectors at or above nvec_max are not stored. */
static void rms_row(const uint16_t* x, const uint16_t* gamma, uint16_t* o, int h, int nt,
                    int nvec_max) {
  float* part = (float*)calloc((size_t)nt, sizeof(float));
  const int vec = (h & 7) == 0;
  for (int tid = 0; tid < nt; ++tid) {
    float s = 0.0f;
    if (vec) {
      for (int u = tid; u < nvec_max; u += nt)
        for (int k = 0; k < 8; ++k) {
          const float f = k3o_bf2f(x[8 * u + k]);
          s = fmaf(f, f, s);
        }
    } else {
      for (int i = tid; i < h; i += nt) {
        const float f = k3o_bf2f(x[i]);
        s = fmaf(f, f, s);
      }
    }
    part[tid] = s;
  }
  const float r = 1.0f / sqrtf(block_sum(part, nt) / (float)h + RMS_EPS);
  const int nout = vec ? 8 * nvec_max : h;
  for (int i = 0; i < nout; ++i)
    o[i] = k3o_f2bf(land(k3o_bf2f(x[i]) * r) * k3o_bf2f(gamma[i]));
  free(part);
}

/* kern_k3_rms (k3_land.cu:104-165): block 1024, every vector of the row. */
void k3o_rms(const uint16_t* x, const uint16_t* gamma, uint16_t* o, int h, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b)
    rms_row(x + (size_t)b * h, gamma, o + (size_t)b * h, h, 1024, h >> 3);
}

/* kern_k3_land (k3_land.cu:168-190): o[b, i] = bf16(p[b ldc + off + i]). */
void k3o_land(const float* p, uint16_t* o, int n, int off, int ldc, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < n; ++i) o[(size_t)b * n + i] = k3o_f2bf(p[(size_t)b * ldc + off + i]);
}

/* The SiTU activation of bf16-landed operands, exactly (double), then the f32
 * value the reference lands: (4 tanh(g/4) sigmoid(g)) (25 tanh(u * 0.04f)),
 * with u * 0.04f the reference's f32 product (k3_land.cu:200-207).  The
 * reference evaluates tanh.approx / __expf / __frcp_rn; the kernel under test
 * is held to one bf16 ulp of this value. */
float k3o_situ(float g, float u) {
  const float uy = u * 0.04f;
  const double gate = 4.0 * tanh((double)g * 0.25) * (1.0 / (1.0 + exp(-(double)g)));
  const double up = 25.0 * tanh((double)uy);
  return (float)(gate * up);
}

void k3o_situ_n(const float* g, const float* u, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = k3o_situ(g[i], u[i]);
}

/* kern_k3_land_situ (f32 p, k3_land.cu:211-237) and kern_k3_land_situ_bf16 /
 * kern_k3_situ_bf16 (bf16 p, k3_land_bf16.cu:56-81, k3_situ_bf16.cu:9-26):
 * row b of p is gate [n] | up [n]; act [B, n]. */
void k3o_land_situ(const float* p_f32, const uint16_t* p_bf16, uint16_t* act, int n, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < n; ++i) {
      const size_t gi = (size_t)b * 2 * n + i, ui = gi + n;
      const float g = p_f32 ? land(p_f32[gi]) : k3o_bf2f(p_bf16[gi]);
      const float u = p_f32 ? land(p_f32[ui]) : k3o_bf2f(p_bf16[ui]);
      act[(size_t)b * n + i] = k3o_f2bf(k3o_situ(g, u));
    }
}

/* kern_k3_situ_rms_bf16 (k3_land_fused.cu:151-202) over a grid of
 * 3 ceil(tokens/16) blocks of 512: situ rows < min(B, 4 ceil(tokens/16)),
 * rms rows < min(L, 4 ceil(tokens/16)) with one vector per thread of 512
 * (vectors past 512 are neither summed nor stored; h % 8 != 0 stores nothing). */
void k3o_situ_rms(const uint16_t* sp, uint16_t* act, const uint16_t* lat, const uint16_t* gam,
                  uint16_t* ln, int n, int B, int h, int L, int tokens) {
  const int cover = 4 * ((tokens + 15) / 16);
  const int bs = B < cover ? B : cover, ls = L < cover ? L : cover;
  k3o_land_situ(NULL, sp, act, n, bs);
  if ((h & 7) != 0) return;
  const int nvec = (h >> 3) < 512 ? (h >> 3) : 512;
#pragma omp parallel for schedule(static)
  for (int b = 0; b < ls; ++b) rms_row(lat + (size_t)b * h, gam, ln + (size_t)b * h, h, 512, nvec);
}
