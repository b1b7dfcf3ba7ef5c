// SiTU gated activation shared by the landing kernels and the MoE fc1 epilogue:
//   situ(g, u) = (alpha tanh(g / alpha) sigmoid(g)) * (beta tanh(u / beta))
// with alpha = 4, beta = 25 in every K3 layer (the manifests fill the per-expert
// moe.alpha / moe.beta buffers with 4.0 and 25.0; k3_land.cu:29-34 hard-codes
// them with u scaled by the f32 constant 0.04f, which equals 1.0f / 25.0f).
// tanh and the logistic come from the hardware 2^x and reciprocal (v_exp_f32,
// v_rcp_f32), with odd Taylor series near 0 where 1 - e^-2x would cancel.
#pragma once
#include "../common/k3_dev.h"

#define K3_LOG2E 0x1.715476p+0f

// ---------------------------------------------------------------- SiTU math
// Per-lane select c ? t : f of two values already computed: the conditional
// operator over expressions is emitted as a branch (the arms' arithmetic sunk
// into it, under an exec mask when the condition diverges), which runs every
// activation as its own short dependent sequence; over two named values it is
// one select (v_cndmask_b32).
K3_DEV float k3_vsel(bool c, float t, float f) { return c ? t : f; }

// tanh(y) for |y| < 0.25: y + y^3 (-1/3 + y^2 (2/15 + y^2 (-17/315 + y^2 62/2835)));
// the first omitted term is below 2^-27 |y| there.
K3_DEV float k3_tanh_series(float y) {
  const float y2 = y * y;
  float p = __builtin_fmaf(y2, 0x1.664f48p-6f, -0x1.ba1ba2p-5f);  // 62/2835, -17/315
  p = __builtin_fmaf(p, y2, 0x1.111112p-3f);                        // 2/15
  p = __builtin_fmaf(p, y2, -0x1.555556p-2f);                       // -1/3
  return __builtin_fmaf(p * y2, y, y);
}

// 4 tanh(g / 4) * sigmoid(g) from t = e^(-|g| / 2) and tt = t^2 = e^-|g|:
//   tanh(|g| / 4) = (1 - t) / (1 + t),  sigmoid(g) = s / (1 + tt), s = 1 (g >= 0)
//   or tt (g < 0), so with r = 1 / ((1 + t)(1 + tt)) (one reciprocal)
//   result = sign(g) s r m,  m = 4 (1 - t),
// or, for |g| < 1 where 1 - t cancels, m = (1 + t) 4 tanh(|g| / 4) from the odd
// series x (1 - x^2 / 48 + x^4 / 1920 - 17 x^6 / 1290240) (x = |g|; the first
// omitted term is below 2^-21 relative).
// SEL true: both m are evaluated and one selected per lane (k3_vsel), the form
// for code that needs the activations' instruction-level parallelism (the fc1
// epilogue, two waves per SIMD: 7% faster); false: the conditional operator
// over the two expressions, which the compiler lowers to exec-masked branches
// (the landing kernels, eight waves per SIMD: measured 15% faster in this form).
// Both forms compute the same values.
template <bool SEL = true>
K3_DEV float k3_situ_gate(float g) {
  const float x = __builtin_fabsf(g);
  const float t = __builtin_amdgcn_exp2f(x * (-0.5f * K3_LOG2E));
  const float tt = t * t;
  const float a = 1.0f + t;
  const float r = __builtin_amdgcn_rcpf(a * (1.0f + tt));
  const float x2 = x * x;
  float p = __builtin_fmaf(x2, -17.0f / 1290240.0f, 1.0f / 1920.0f);
  p = __builtin_fmaf(p, x2, -1.0f / 48.0f);
  p = __builtin_fmaf(p, x2, 1.0f);
  float m;
  if constexpr (SEL) m = k3_vsel(x < 1.0f, p * x * a, __builtin_fmaf(-4.0f, t, 4.0f));
  else m = x < 1.0f ? p * x * a : __builtin_fmaf(-4.0f, t, 4.0f);
  const float s = g >= 0.0f ? 1.0f : tt;
  return __builtin_copysignf(m * s * r, g);
}

// 25 tanh(u * 0.04) (the reference scales by the f32 constant 0.04f): with
// x = |u * 0.04| and e = e^(-2 x), 25 (1 - e) / (1 + e), or for x < 0.25 the odd
// series x (25 - 25 x^2 / 3 + 10 x^4 / 3 - 85 x^6 / 63) (first omitted term
// below 2^-21 relative).  EXPF false: the series alone, the same value wherever
// x < 0.25, for callers that have established that for every active lane
// (k3_situ_up_series_ok).  SEL as for k3_situ_gate.
template <bool SEL = true, bool EXPF = true>
K3_DEV float k3_situ_up(float u) {
  const float y = u * 0.04f;
  const float x = __builtin_fabsf(y);
  const float x2 = x * x;
  float p = __builtin_fmaf(x2, -85.0f / 63.0f, 10.0f / 3.0f);
  p = __builtin_fmaf(p, x2, -25.0f / 3.0f);
  p = __builtin_fmaf(p, x2, 25.0f);
  if constexpr (!EXPF) return __builtin_copysignf(p * x, y);
  const float e = __builtin_amdgcn_exp2f(x * (-2.0f * K3_LOG2E));
  float th;
  if constexpr (SEL)
    th = k3_vsel(x < 0.25f, p * x,
                 __builtin_fmaf(-25.0f, e, 25.0f) * __builtin_amdgcn_rcpf(1.0f + e));
  else
    th = x < 0.25f ? p * x : __builtin_fmaf(-25.0f, e, 25.0f) * __builtin_amdgcn_rcpf(1.0f + e);
  return __builtin_copysignf(th, y);
}

// Wave-uniform: true when every active lane's |u * 0.04| < 0.25 for each u
// with |u| <= umax (umax: the lane's largest |u|, NaN treated as needing the
// exponential form; fl(|u| * 0.04) is monotone in |u|), so that k3_situ_up<false>
// gives every lane's value.
K3_DEV bool k3_situ_up_series_ok(float umax) {
  return __builtin_amdgcn_ballot_w64(!(umax * 0.04f < 0.25f)) == 0;
}

template <bool SEL = true, bool EXPF = true>
K3_DEV float k3_situ(float g, float u) {
  return k3_situ_gate<SEL>(g) * k3_situ_up<SEL, EXPF>(u);
}

// k3_situ with one reciprocal for the two factors' denominators: with t, tt, m,
// s of k3_situ_gate and e = e^(-2 |u * 0.04|),
//   situ = sign(g) sign(u) (m s) (n / ((1 + t)(1 + tt)(1 + e))),
//   n = 25 (1 - e), or for |u * 0.04| < 0.25 the series of k3_situ_up times (1 + e),
// three transcendentals instead of four (the fc1 epilogue, bound by its vector
// ALU: measured 2% of fc1).  The same bound as k3_situ: relative error below
// 4e-6, checked against double precision over every 13th f32 g in [2^-20, 200]
// of both signs crossed with 20 values of u across the series boundary, and the
// converse.  EXPF false as for k3_situ_up.
template <bool EXPF = true>
K3_DEV float k3_situ_fused(float g, float u) {
  const float x = __builtin_fabsf(g);
  const float t = __builtin_amdgcn_exp2f(x * (-0.5f * K3_LOG2E));
  const float tt = t * t;
  const float a = 1.0f + t;
  const float x2 = x * x;
  float p = __builtin_fmaf(x2, -17.0f / 1290240.0f, 1.0f / 1920.0f);
  p = __builtin_fmaf(p, x2, -1.0f / 48.0f);
  p = __builtin_fmaf(p, x2, 1.0f);
  const float m = k3_vsel(x < 1.0f, p * x * a, __builtin_fmaf(-4.0f, t, 4.0f));
  const float s = g >= 0.0f ? 1.0f : tt;
  const float y = u * 0.04f;
  const float xu = __builtin_fabsf(y);
  const float xu2 = xu * xu;
  float q = __builtin_fmaf(xu2, -85.0f / 63.0f, 10.0f / 3.0f);
  q = __builtin_fmaf(q, xu2, -25.0f / 3.0f);
  q = __builtin_fmaf(q, xu2, 25.0f);
  float n, d = a * (1.0f + tt);
  if constexpr (EXPF) {
    const float e = __builtin_amdgcn_exp2f(xu * (-2.0f * K3_LOG2E));
    const float c = 1.0f + e;
    n = k3_vsel(xu < 0.25f, q * xu * c, __builtin_fmaf(-25.0f, e, 25.0f));
    d = d * c;
  } else {
    n = q * xu;
  }
  const float mag = (m * s) * (n * __builtin_amdgcn_rcpf(d));
  return __uint_as_float(__float_as_uint(mag) ^
                         ((__float_as_uint(g) ^ __float_as_uint(y)) & 0x80000000u));
}

// General alpha / beta (per expert).  inv_alpha = 1 / alpha and inv_beta =
// 1 / beta (correctly rounded); for alpha == 4 callers take k3_situ_gate (the
// fc1 epilogue chooses per item).  Every form here is within a few f32 ulp of
// the exact activation (relative error below 4e-6, checked against double
// precision over all f32 inputs in [2^-20, 200]); the fc1 epilogue takes
// k3_situ when alpha == 4 and beta == 25.
K3_DEV float k3_situ_gate_a(float g, float alpha, float inv_alpha) {
  const float x = __builtin_fabsf(g);
  const float y = x * inv_alpha;
  const float e = __builtin_amdgcn_exp2f(y * (-2.0f * K3_LOG2E));
  const float th =
      k3_vsel(y < 0.25f, k3_tanh_series(y), (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e));
  const float t2 = __builtin_amdgcn_exp2f(x * -K3_LOG2E);  // e^-|g|
  const float r = __builtin_amdgcn_rcpf(1.0f + t2);
  const float sg = g >= 0.0f ? r : t2 * r;
  return __builtin_copysignf(alpha * th, g) * sg;
}

// EXPF false: the series alone (k3_situ_up_b_series_ok), as k3_situ_up.
template <bool EXPF = true>
K3_DEV float k3_situ_up_b(float u, float beta, float inv_beta) {
  const float y = u * inv_beta;
  const float x = __builtin_fabsf(y);
  if constexpr (!EXPF) return beta * __builtin_copysignf(k3_tanh_series(x), y);
  const float e = __builtin_amdgcn_exp2f(x * (-2.0f * K3_LOG2E));
  const float th =
      k3_vsel(x < 0.25f, k3_tanh_series(x), (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e));
  return beta * __builtin_copysignf(th, y);
}

K3_DEV bool k3_situ_up_b_series_ok(float umax, float inv_beta) {
  return __builtin_amdgcn_ballot_w64(!(__builtin_fabsf(umax * inv_beta) < 0.25f)) == 0;
}
