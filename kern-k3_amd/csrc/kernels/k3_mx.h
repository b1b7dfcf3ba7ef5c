// MXFP8 (OCP e4m3 payload, E8M0 block scale, 32-element blocks) helpers.
//
// Block semantics (reference kern_k3_moe_quant, k3_moe_prefill_v4.cu:111-140):
//   amax = max |x| over the 32 values (f32 max, NaN ignored);
//   e    = amax > 0 ? clamp(ceil(log2(amax / 448)), -127, 127) : 0;
//   sf   = e + 127;  q = e4m3_rne_satfinite(x * 2^-e).
// Every finite x satisfies |x * 2^-e| <= amax * 2^-e <= 448, so the conversion
// never saturates and the hardware RNE conversion gives the payload directly.
//
// Work split: a 32-value block is held by four consecutive lanes (a DPP quad),
// eight bf16 (16 bytes) each; the block amax is a two-step quad max of the
// |bf16| bit patterns (monotone in the magnitude for non-NaN values).
#pragma once
#include "../common/k3_dev.h"

// Largest |bf16| pattern (NaN excluded) of the eight values of one 16-byte vector.
K3_DEV uint32_t k3_vec_absmax_bits(k3_u4 v) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = k3_absbits_nonan(v[j] & 0xffffu);
    const uint32_t hi = k3_absbits_nonan(v[j] >> 16);
    m = m > lo ? m : lo;
    m = m > hi ? m : hi;
  }
  return m;
}

// Scale eight bf16 by 2^-e and convert to e4m3: two words, byte k = value k.
// e4m3 codes of eight values already in f32 (x * 2^-e for the block exponent e;
// x bf16-representable), in order.
K3_DEV k3_u2 k3_f8_to_e4m3(const float (&x)[8], int e) {
  float f[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) f[k] = __builtin_ldexpf(x[k], -e);
  k3_u2 o;
  o[0] = k3_pack_e4m3x4(f[0], f[1], f[2], f[3]);
  o[1] = k3_pack_e4m3x4(f[4], f[5], f[6], f[7]);
  if (e == 127) {
    // Only a block holding +-inf reaches e = 127; the saturating conversion
    // maps +-inf to +-448 (0x7e / 0xfe), which the plain conversion does not.
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (__builtin_isinf(f[k])) {
        const uint32_t code = 0x7eu | (f[k] < 0.0f ? 0x80u : 0u);
        const int w = k >> 2, sh = (k & 3) * 8;
        o[w] = (o[w] & ~(0xffu << sh)) | (code << sh);
      }
    }
  }
  return o;
}

K3_DEV k3_u2 k3_vec_to_e4m3(k3_u4 v, int e) {
  float x[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = k3_bf_lo(v[j]);
    x[2 * j + 1] = k3_bf_hi(v[j]);
  }
  return k3_f8_to_e4m3(x, e);
}

// Quantise the 16-byte vector this lane holds; the quad's block exponent is
// returned (all four lanes agree).  Every lane of the quad must execute this.
K3_DEV int k3_mx_quad(k3_u4 v, k3_u2* q) {
  const uint32_t m = k3_quad_max_u32(k3_vec_absmax_bits(v));
  const int e = k3_e8m0_exp(m);
  *q = k3_vec_to_e4m3(v, e);
  return e;
}
