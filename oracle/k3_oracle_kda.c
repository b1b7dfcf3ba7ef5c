/* CPU oracle, part 3: KDA short-conv span gather and output gate.
 * TEST INFRASTRUCTURE ONLY (see k3_oracle.h). */
#include <math.h>
#include <string.h>

#include "k3_oracle.h"

static inline float land(float f) { return k3o_bf2f(k3o_f2bf(f)); }

/* kern_k3_span_gather (k3_span_gather_v3.cu:251-293; contract
 * k3_span_gather_v2.cu:10-31).  win holds the three streams' windows
 * [3 stream][3 row][inner] bf16 and is updated in place to the last three
 * inputs; rows [at, at + span) of partial / wsm are read.  The conv is the fma
 * chain fma(x_i, w3, fma(x_{i-1}, w2, fma(x_{i-2}, w1, x_{i-3} w0))); the SiLU
 * is sb * 1 / (1 + e^-sb) with the deterministic exp (the reference uses the
 * ex2.approx / rcp.approx forms, within one bf16 ulp after the landing). */
void k3o_span_gather(const uint16_t* partial, const float* cw, uint16_t* win, const float* wsm,
                     uint16_t* span_q, uint16_t* span_k, uint16_t* span_v, uint16_t* span_beta,
                     uint16_t* span_flow, int at, int span, int heads) {
  const int inner = heads * 128, fused = 4 * inner;
  uint16_t* outs[3] = {span_q, span_k, span_v};
  for (int s = 0; s < 3; ++s) {
    uint16_t* wn = win + (size_t)s * 3 * inner;
    uint16_t* out = outs[s];
#pragma omp parallel for schedule(static)
    for (int c = 0; c < inner; ++c) {
      const float w0 = cw[((size_t)s * 4 + 0) * inner + c], w1 = cw[((size_t)s * 4 + 1) * inner + c];
      const float w2 = cw[((size_t)s * 4 + 2) * inner + c], w3 = cw[((size_t)s * 4 + 3) * inner + c];
      float t0 = k3o_bf2f(wn[c]), t1 = k3o_bf2f(wn[inner + c]), t2 = k3o_bf2f(wn[2 * inner + c]);
      for (int i = 0; i < span; ++i) {
        const float x = k3o_bf2f(partial[(size_t)(at + i) * fused + (size_t)s * inner + c]);
        float y = t0 * w0;
        y = fmaf(t1, w1, y);
        y = fmaf(t2, w2, y);
        y = fmaf(x, w3, y);
        const float sb = land(y);
        out[(size_t)i * inner + c] = k3o_f2bf(sb * k3o_sigmoid(sb));
        t0 = t1; t1 = t2; t2 = x;
      }
      /* new window: the last three inputs (old window rows when span < 3) */
      const uint16_t nw0 = k3o_f2bf(t0), nw1 = k3o_f2bf(t1), nw2 = k3o_f2bf(t2);
      wn[c] = nw0; wn[inner + c] = nw1; wn[2 * inner + c] = nw2;
    }
  }
  for (int i = 0; i < span; ++i) {
    const float* row = wsm + (size_t)(at + i) * 256;
    for (int h = 0; h < heads; ++h) span_beta[(size_t)h * span + i] = k3o_f2bf(row[h]);
    for (int j = 0; j < 128; ++j) span_flow[(size_t)i * 128 + j] = k3o_f2bf(row[96 + j]);
  }
}

/* kern_k3_kda_out_gate (k3_kda_out_gate_v3.cu:36-118): per (row, head) the sum
 * of squares in the reference order -- 16 lanes with 8 serial fmas each, then
 * a xor butterfly 8, 4, 2, 1 -- r = 1 / sqrt(ss / 128 + eps) (rsqrtf replaced by
 * the correctly rounded form; eps is the module's K11_RMS_EPS, 1e-5 or 1e-6,
 * k3_kda_out_gate_v3.cu:25,92), o = bf16(a r gamma_o), gt = bf16(sigmoid(g)),
 * gated = bf16(o gt).  Rows [at, at + span) of gated are written. */
void k3o_kda_out_gate(const uint16_t* attn, const uint16_t* gate_partial, const float* gamma_o,
                      uint16_t* gated, int at, int span, int heads, float eps) {
  const int inner = heads * 128, fused = 4 * inner;
#pragma omp parallel for schedule(static)
  for (int i = 0; i < span; ++i) {
    const int b = at + i;
    for (int h = 0; h < heads; ++h) {
      float lane[16], tmp[16];
      for (int l = 0; l < 16; ++l) {
        float s = 0.0f;
        for (int k = 0; k < 8; ++k) {
          const float a = k3o_bf2f(attn[(size_t)i * inner + h * 128 + l * 8 + k]);
          s = fmaf(a, a, s);
        }
        lane[l] = s;
      }
      for (int o = 8; o > 0; o >>= 1) {
        for (int l = 0; l < 16; ++l) tmp[l] = lane[l] + lane[l ^ o];
        memcpy(lane, tmp, sizeof(lane));
      }
      const float r = 1.0f / sqrtf(fmaf(lane[0], 1.0f / 128.0f, eps));
      for (int dv = 0; dv < 128; ++dv) {
        const float a = k3o_bf2f(attn[(size_t)i * inner + h * 128 + dv]);
        const float o = land(a * r * gamma_o[dv]);
        const float g = k3o_bf2f(gate_partial[(size_t)b * fused + 3 * inner + h * 128 + dv]);
        const float gt = land(k3o_sigmoid(g));
        gated[(size_t)b * inner + h * 128 + dv] = k3o_f2bf(o * gt);
      }
    }
  }
}
