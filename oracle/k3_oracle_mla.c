/* CPU oracle, part 4: MLA prep (reference ABI) and the latent-norm + RoPE +
 * q packing op.  TEST INFRASTRUCTURE ONLY (see k3_oracle.h). */
#include <math.h>
#include <string.h>

#include "k3_oracle.h"

#define Q_LORA 1536
#define KV_LORA 512
#define ROPE 64
#define KV_A 576
#define HEADC 2112

static inline float land(float f) { return k3o_bf2f(k3o_f2bf(f)); }

static float bfly32(const float* v) {
  float a[32], b[32];
  memcpy(a, v, sizeof(a));
  for (int o = 16; o > 0; o >>= 1) {
    for (int i = 0; i < 32; ++i) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof(a));
  }
  return a[0];
}

/* group partial of 32 float4 units starting at unit u0: each unit's four
 * landed squares summed from 0 (fma), then a 32-lane butterfly
 * (k3_mla_prep_v2.cu:144-168) */
static float group_sq(const float* P, int u0) {
  float p[32];
  for (int l = 0; l < 32; ++l) {
    float s = 0.0f;
    for (int k = 0; k < 4; ++k) { const float x = P[4 * (u0 + l) + k]; s = fmaf(x, x, s); }
    p[l] = s;
  }
  return bfly32(p);
}

/* kern_k3_mla_prep_head + kern_k3_mla_prep_gate (k3_mla_prep_v2.cu:91-211;
 * bf16 twin k3_mla_prep_bf16.cu).  partial_f32 or partial_bf16 (one non-null)
 * [B, mla_fused]; the slab is written at (slot/64)*page_stride + layer_off +
 * (slot%64)*576 (elements) for slot >= 0.  rsqrtf is replaced by the correctly
 * rounded 1 / sqrt. */
void k3o_mla_prep(const float* partial_f32, const uint16_t* partial_bf16, int mla_fused,
                  int inner, const uint16_t* gamma_q_a, const uint16_t* gamma_kv_a,
                  const long long* slot_mapping, uint16_t* slab, long long layer_off,
                  long long page_stride, uint16_t* q_norm, uint16_t* mla_gate, int B) {
#pragma omp parallel for schedule(static)
  for (int b = 0; b < B; ++b) {
    float P[HEADC];
    for (int i = 0; i < HEADC; ++i)
      P[i] = partial_bf16 ? k3o_bf2f(partial_bf16[(size_t)b * mla_fused + i])
                          : land(partial_f32[(size_t)b * mla_fused + i]);
    float tq = 0.0f, tk = 0.0f;
    for (int g = 0; g < 12; ++g) tq += group_sq(P, 32 * g);
    for (int g = 0; g < 4; ++g) tk += group_sq(P, Q_LORA / 4 + 32 * g);
    const float scq = 1.0f / sqrtf(fmaf(tq, 1.0f / Q_LORA, 1e-5f));
    const float sck = 1.0f / sqrtf(fmaf(tk, 1.0f / KV_LORA, 1e-5f));
    for (int i = 0; i < Q_LORA; ++i)
      q_norm[(size_t)b * Q_LORA + i] = k3o_f2bf(land(P[i] * scq) * k3o_bf2f(gamma_q_a[i]));
    const long long slot = slot_mapping[b];
    if (slot >= 0) {
      uint16_t* rowp = slab + (slot / 64) * page_stride + layer_off + (slot % 64) * KV_A;
      for (int i = 0; i < KV_LORA; ++i)
        rowp[i] = k3o_f2bf(land(P[Q_LORA + i] * sck) * k3o_bf2f(gamma_kv_a[i]));
      for (int i = 0; i < ROPE; ++i) rowp[KV_LORA + i] = k3o_f2bf(P[Q_LORA + KV_LORA + i]);
    }
    for (int i = 0; i < inner; ++i) {
      const size_t o = (size_t)b * mla_fused + HEADC + i;
      mla_gate[(size_t)b * inner + i] =
          partial_bf16 ? partial_bf16[o] : k3o_f2bf(partial_f32[o]);
    }
  }
}

/* Latent RMSNorm + interleaved RoPE + q packing (no reference entry).  Sum of
 * squares: 64 lanes of 8 serial fmas, 64-lane xor butterfly; cos / sin are the
 * f32 roundings of the double cos / sin of p * theta^(-2j/64); rotation
 * y0 = fma(x0, c, -(x1 s)), y1 = fma(x0, s, x1 c), one bf16 landing. */
void k3o_mla_rope_pack(const uint16_t* latent, const uint16_t* k_rope, const uint16_t* q,
                       const uint16_t* gamma_kv, const long long* positions, uint16_t* latent_out,
                       uint16_t* q_out, float theta, float eps, int T, int H) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    float c[32], s[32];
    for (int j = 0; j < 32; ++j) {
      const double inv = pow((double)theta, -(double)(2 * j) / 64.0);
      const double ang = (double)positions[t] * inv;
      c[j] = (float)cos(ang);
      s[j] = (float)sin(ang);
    }
    float lane[64], tmp[64];
    for (int l = 0; l < 64; ++l) {
      float a = 0.0f;
      for (int k = 0; k < 8; ++k) {
        const float x = k3o_bf2f(latent[(size_t)t * KV_LORA + 8 * l + k]);
        a = fmaf(x, x, a);
      }
      lane[l] = a;
    }
    for (int o = 32; o > 0; o >>= 1) {
      for (int l = 0; l < 64; ++l) tmp[l] = lane[l] + lane[l ^ o];
      memcpy(lane, tmp, sizeof(lane));
    }
    const float r = 1.0f / sqrtf(fmaf(lane[0], 1.0f / KV_LORA, eps));
    uint16_t* lrow = latent_out + (size_t)t * KV_A;
    for (int i = 0; i < KV_LORA; ++i)
      lrow[i] = k3o_f2bf(land(k3o_bf2f(latent[(size_t)t * KV_LORA + i]) * r) * k3o_bf2f(gamma_kv[i]));
    for (int j = 0; j < 32; ++j) {
      const float x0 = k3o_bf2f(k_rope[(size_t)t * ROPE + 2 * j]);
      const float x1 = k3o_bf2f(k_rope[(size_t)t * ROPE + 2 * j + 1]);
      lrow[KV_LORA + 2 * j] = k3o_f2bf(fmaf(x0, c[j], -(x1 * s[j])));
      lrow[KV_LORA + 2 * j + 1] = k3o_f2bf(fmaf(x0, s[j], x1 * c[j]));
    }
    for (int h = 0; h < H; ++h) {
      const uint16_t* qi = q + ((size_t)t * H + h) * 192;
      uint16_t* qo = q_out + ((size_t)t * H + h) * 192;
      memcpy(qo, qi, 128 * sizeof(uint16_t));
      for (int j = 0; j < 32; ++j) {
        const float x0 = k3o_bf2f(qi[128 + 2 * j]), x1 = k3o_bf2f(qi[128 + 2 * j + 1]);
        qo[128 + 2 * j] = k3o_f2bf(fmaf(x0, c[j], -(x1 * s[j])));
        qo[128 + 2 * j + 1] = k3o_f2bf(fmaf(x0, s[j], x1 * c[j]));
      }
    }
  }
}
