// Device-side numeric and cross-lane primitives shared by every gfx950 module.
//
// Conventions
// -----------
// * bf16 values travel as raw 16-bit patterns (the upper half of an f32).  A
//   bf16 -> f32 widening is a shift; f32 -> bf16 is the gfx950 instruction
//   v_cvt_pk_bf16_f32 (round to nearest even, two values per instruction).
// * e4m3 payloads are OCP FP8 E4M3 ("fn": no infinities, 0x7f/0xff = NaN,
//   largest finite 448) produced by v_cvt_pk_fp8_f32 (round to nearest even),
//   with every NaN code made the canonical 0x7f of the saturating conversion.
// * Every module is compiled with -ffp-contract=off: a fused multiply-add
//   appears only where it is written as __builtin_fmaf, so the CPU checker
//   can reproduce each sum bit for bit.
// * Cross-lane sums reproduce a 32-lane xor butterfly (offsets 16, 8, 4, 2, 1)
//   inside each half of the 64-lane wavefront.  Both partners of an xor pair
//   add the same two numbers, so every lane of a 32-lane group ends with the
//   same bits, and the association is the one the reference kernels' warp
//   reductions use (k3_residual_v2.cu:92-96).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define K3_DEV __device__ __forceinline__

typedef float k3_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 k3_bf2 __attribute__((ext_vector_type(2)));
typedef uint32_t k3_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t k3_u2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- bf16
K3_DEV float k3_bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
K3_DEV float k3_bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
K3_DEV float k3_bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Two f32 -> one word of two bf16 (lo in bits 0..15), RNE.
K3_DEV uint32_t k3_pack_bf2(float lo, float hi) {
  k3_f2 f = {lo, hi};
  k3_bf2 b = __builtin_convertvector(f, k3_bf2);
  return __builtin_bit_cast(uint32_t, b);
}

// f32 -> bf16 -> f32 (the "landing" of one value).
K3_DEV float k3_land(float x) {
  return k3_bf_lo(k3_pack_bf2(x, 0.0f));
}

// bf16 x bf16 -> bf16 for a packed pair: the product of two 8-bit significands
// is exact in f32, so one RNE rounding of the f32 product is the result.
K3_DEV uint32_t k3_mul_bf2(uint32_t a, uint32_t g) {
  return k3_pack_bf2(k3_bf_lo(a) * k3_bf_lo(g), k3_bf_hi(a) * k3_bf_hi(g));
}

// ---------------------------------------------------------------- e4m3
// NaN codes of a word of four e4m3 bytes made canonical: v_cvt_pk_fp8_f32
// turns a NaN input into 0xff whatever its sign, the saturating conversion of
// the reference kernels (__nv_cvt_float_to_fp8 with __NV_SATFINITE) into 0x7f.
// A byte is NaN exactly when its low seven bits are all ones; adding 1 to those
// seven bits carries into bit 7 only then (never into the next byte), and that
// carry clears the byte's sign bit.
K3_DEV uint32_t k3_e4m3_nan_canon(uint32_t w) {
  return w & ~(((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u);
}
// Two f32 -> two e4m3 bytes in the low half of the result (byte 0 = a).
K3_DEV uint32_t k3_pack_e4m3x2(float a, float b) {
  return k3_e4m3_nan_canon((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu);
}
// Four f32 -> one word of four e4m3 bytes (byte k = value k).
K3_DEV uint32_t k3_pack_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return k3_e4m3_nan_canon((uint32_t)w);
}

// E8M0 block exponent of a block whose largest |value| has the bf16 bit
// pattern `amax_bits` (sign already cleared, NaN patterns excluded by the
// caller): e = clamp(ceil(log2(amax / 448)), -127, 127), 0 when amax == 0.
// With amax = M * 2^E, M in [1, 2): 448 = 1.75 * 2^8, so
// log2(amax / 448) = E - 8 + log2(M / 1.75), and log2(M / 1.75) lies in
// (-1, 0] for M <= 1.75 and in (0, 1) above; for a bf16 M the quotient is never
// within f32 rounding of a power of two except at M == 1.75 exactly.  Hence
// e = E - 8 + (M > 1.75).  +inf (0x7f80) gives +inf through ceil(log2(.)) and
// saturates to 127.  bf16 subnormals have E <= -127 and clamp to -127.
K3_DEV int k3_e8m0_exp(uint32_t amax_bits) {
  if (amax_bits == 0u) return 0;
  if (amax_bits >= 0x7f80u) return 127;
  const int E = (int)(amax_bits >> 7) - 127;
  int e = E - 8 + (((amax_bits & 0x7fu) > 0x60u) ? 1 : 0);
  e = e < -127 ? -127 : e;
  return e;
}

// |bf16| bit pattern for the amax of an MX block: NaN patterns count as 0
// (the f32 max the block scale is defined by ignores NaN operands).
K3_DEV uint32_t k3_absbits_nonan(uint32_t h16) {
  const uint32_t a = h16 & 0x7fffu;
  return a > 0x7f80u ? 0u : a;
}

// ---------------------------------------------------------------- cross-lane
// DPP quad permutations (lanes 4k..4k+3).
#define K3_DPP_QP_1032 0xb1  // quad_perm [1,0,3,2]
#define K3_DPP_QP_2301 0x4e  // quad_perm [2,3,0,1]

K3_DEV uint32_t k3_quad_max_u32(uint32_t v) {
  uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_1032, 0xf, 0xf, false);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_QP_2301, 0xf, 0xf, false);
  return v > o ? v : o;
}

// Wave-wide unsigned max, returned uniform.  GFX9 DPP: quad exchanges, then
// the half-row and row mirrors make every lane of a 16-lane row hold the row
// max; row_bcast15 folds row 0 into row 1 and row 2 into row 3, row_bcast31
// folds rows 0-1 into row 3, whose lane 63 then holds the wave max.  Lanes a
// broadcast does not write keep 0, the identity of the max.
#define K3_DPP_ROW_MIRROR 0x140
#define K3_DPP_ROW_HALF_MIRROR 0x141
#define K3_DPP_ROW_BCAST15 0x142
#define K3_DPP_ROW_BCAST31 0x143

K3_DEV uint32_t k3_wave_max_u32_uniform(uint32_t v) {
  v = k3_quad_max_u32(v);
  uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_HALF_MIRROR, 0xf, 0xf, false);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K3_DPP_ROW_MIRROR, 0xf, 0xf, false);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K3_DPP_ROW_BCAST15, 0xa, 0xf, false);
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K3_DPP_ROW_BCAST31, 0xc, 0xf, false);
  v = v > o ? v : o;
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// xor swizzle inside 32-lane groups (ds_swizzle bit mode: and 0x1f, xor m).
template <int M>
K3_DEV float k3_swz_xor(float v) {
  static_assert(M > 0 && M < 32, "xor mask within 32 lanes");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (M << 10)));
}
template <int M>
K3_DEV uint32_t k3_swz_xor_u32(uint32_t v) {
  static_assert(M > 0 && M < 32, "xor mask within 32 lanes");
  return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1f | (M << 10));
}

// Sum over each 32-lane group in butterfly order 16, 8, 4, 2, 1.
K3_DEV float k3_sum32(float v) {
  v += k3_swz_xor<16>(v);
  v += k3_swz_xor<8>(v);
  v += k3_swz_xor<4>(v);
  v += k3_swz_xor<2>(v);
  v += k3_swz_xor<1>(v);
  return v;
}
// Sum over each 16-lane group in butterfly order 8, 4, 2, 1.
K3_DEV float k3_sum16(float v) {
  v += k3_swz_xor<8>(v);
  v += k3_swz_xor<4>(v);
  v += k3_swz_xor<2>(v);
  v += k3_swz_xor<1>(v);
  return v;
}
K3_DEV float k3_max32(float v) {
  v = fmaxf(v, k3_swz_xor<16>(v));
  v = fmaxf(v, k3_swz_xor<8>(v));
  v = fmaxf(v, k3_swz_xor<4>(v));
  v = fmaxf(v, k3_swz_xor<2>(v));
  v = fmaxf(v, k3_swz_xor<1>(v));
  return v;
}

// ---------------------------------------------------------------- math
// Deterministic exp(x): Cody-Waite reduction x = n ln2 + r with a two-part ln2
// (the high part has 12 trailing zero bits so n * ln2_hi is exact for
// |n| < 2^12), e^r by the degree-7 Taylor polynomial in Horner form with
// explicit fma, then a scaling by 2^n.  Every step is a correctly rounded f32
// operation, so the CPU checker computes the same bits.  Valid for
// x in [-87, 88]; callers clamp.  Relative error about 1 ulp.
K3_DEV float k3_expf(float x) {
  const float n = __builtin_rintf(x * 0x1.715476p+0f);       // log2(e)
  float r = __builtin_fmaf(n, -0x1.62e4p-1f, x);              // ln2 high part
  r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);                 // ln2 low part
  float p = 0x1.a01a02p-13f;                                  // 1/7!
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);                  // 1/6!
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);                   // 1/5!
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);                   // 1/4!
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);                   // 1/3!
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// Deterministic logistic function 1 / (1 + e^-x) with IEEE division.  With
// t = -x: t >= 0x1.62e430p+6 overflows e^t in f32, giving 1 / (1 + inf) = 0;
// below -87, 1 + e^t is exactly 1, so t is clamped there.  NaN propagates.
K3_DEV float k3_sigmoid(float x) {
  const float t = -x;
  if (t >= 0x1.62e430p+6f) return 0.0f;
  return 1.0f / (1.0f + k3_expf(t < -87.0f ? -87.0f : t));
}

// k3_sigmoid without a branch (same bits for every input, NaN included): the
// overflow side is evaluated on a clamped argument and selected away.
K3_DEV float k3_sigmoid_nb(float x) {
  const float t = -x;
  const bool over = t >= 0x1.62e430p+6f;
  const float tc = over ? 0.0f : (t < -87.0f ? -87.0f : t);
  const float r = 1.0f / (1.0f + k3_expf(tc));
  return over ? 0.0f : r;
}

// Fast logistic for bf16-landed inputs: hardware 2^x and reciprocal
// (v_exp_f32, v_rcp_f32), about 1 ulp each; results are rounded to bf16.
K3_DEV float k3_sigmoid_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -0x1.715476p+0f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// Correctly rounded 1 / sqrt(v): IEEE sqrt then IEEE division (the build
// compiles with correctly rounded f32 divide and sqrt).
K3_DEV float k3_rsqrt_cr(float v) { return 1.0f / __builtin_sqrtf(v); }

// Order-preserving f32 -> u32 key (total order on non-NaN values).
K3_DEV uint32_t k3_ord_f32(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------- memory
K3_DEV k3_u4 k3_ld16(const void* p) { return *(const k3_u4*)p; }
K3_DEV void k3_st16(void* p, k3_u4 v) { *(k3_u4*)p = v; }
K3_DEV k3_u4 k3_ld16_nt(const void* p) { return __builtin_nontemporal_load((const k3_u4*)p); }
K3_DEV void k3_st16_nt(void* p, k3_u4 v) { __builtin_nontemporal_store(v, (k3_u4*)p); }
K3_DEV void k3_st8_nt(void* p, k3_u2 v) { __builtin_nontemporal_store(v, (k3_u2*)p); }
// Non-temporal store through an address read from memory (a peer rank's
// buffer): cast to the global address space, so it is issued as a global store
// and counts only in the vector memory counter.  Through the generic pointer it
// would be a flat store, which also counts in the counter that scalar loads
// wait on, so the wait for the next peer address would wait for the store.
typedef __attribute__((address_space(1))) k3_u4 k3_gu4;
K3_DEV void k3_st16_nt_g(void* p, k3_u4 v) { __builtin_nontemporal_store(v, (k3_gu4*)p); }
K3_DEV float4 k3_ld16f_nt(const float* p) {
  const k3_u4 u = k3_ld16_nt(p);
  return make_float4(__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]), __uint_as_float(u[3]));
}
