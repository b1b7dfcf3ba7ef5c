// Modules k3_mla_prep_v2+INNER=3072+MLA_FUSED=5184 (f32 partial) and
// k3_mla_prep_bf16+INNER=3072+MLA_FUSED=5184 (bf16 partial, K3_MLA_BF16): MLA prep (K4).
//
//   kern_k3_mla_prep_head(partial, gamma_q_a, gamma_kv_a, slot_mapping, slab, layer_off,
//                         page_stride, q_norm, B)          grid ceil(B/4), block 512
//   kern_k3_mla_prep_gate(partial, mla_gate, B)            grid ceil(B/4), block 384
//   k3h_mla_prep_fused(partial, gamma_q_a, gamma_kv_a, slot_mapping, slab, layer_off,
//                      page_stride, q_norm, mla_gate, B)   grid ceil(B/4), block 512
//
// Entries, parameters and geometry are the reference's (k3_mla_prep_v2.cu:91,130;
// k3_mla_prep_bf16.cu:73,112; manifest op mla_prep, k3-tp4-prefill-16k.json:404677,
// page_stride 884736).  Row b of the fused partial is
// [q_a 1536 | kv_a 512 | rope 64 | gate INNER], every value landed to bf16 first:
//   q_norm[b]  = bf16(bf16(q_a * rsqrt(mean(q_a^2) + 1e-5)) (x) gamma_q_a)
//   kv_norm    = the same over kv_a with gamma_kv_a
//   slab[(slot/64)*page_stride + layer_off + (slot%64)*576 + 0..512) = kv_norm,
//        + 512..576 = bf16(rope); skipped when slot_mapping[b] < 0
//   mla_gate[b] = bf16(P[b, 2112 .. 2112 + INNER))
// Sum-of-squares order (k3_mla_prep_v2.cu:120-179): the row's float4 units are
// cut into 12 q groups and 4 kv groups of 32 units; a unit's four landed squares
// are summed from 0, a group is a 32-lane xor butterfly, and the group partials
// are added in group order.  Four 128-thread row slices per workgroup; a slice's
// half-wave `sub` owns q groups 3 sub .. 3 sub + 2 and kv group sub.
#include "../common/k3_dev.h"

#define Q_LORA 1536
#define KV_LORA 512
#define ROPE 64
#define KV_A (KV_LORA + ROPE)
#define HEADC (Q_LORA + KV_LORA + ROPE)
#ifndef INNER
#define INNER 3072
#endif
#ifndef MLA_FUSED
#define MLA_FUSED (HEADC + INNER)
#endif
#define EPSV 1e-5f
#define QU (Q_LORA / 4)
#define KU ((Q_LORA + KV_LORA) / 4)
#define PG_THREADS 384
#define PG_ROWS 4
#define PG_COLS (INNER / PG_THREADS)
#define PH_ROWS 4
#define PH_THREADS (PH_ROWS * 128)
static_assert(INNER % 1024 == 0, "gate columns: whole 16-byte vectors per thread of a row slice");
#ifndef MLA_NT
#define MLA_NT 1  // partial rows are read once: non-temporal loads
#endif

#ifdef K3_MLA_BF16
typedef uint16_t k3_mla_t;
// four consecutive partial values of a row, landed (bf16 input: exact)
K3_DEV float4 k3_mla_ld4(const k3_mla_t* p) {
#if MLA_NT
  const k3_u2 w = __builtin_nontemporal_load((const k3_u2*)p);
#else
  const k3_u2 w = *(const k3_u2*)p;
#endif
  return make_float4(k3_bf_lo(w[0]), k3_bf_hi(w[0]), k3_bf_lo(w[1]), k3_bf_hi(w[1]));
}
#else
typedef float k3_mla_t;
K3_DEV float4 k3_mla_ld4(const k3_mla_t* p) {
#if MLA_NT
  const k3_u4 u = k3_ld16_nt(p);
#else
  const k3_u4 u = k3_ld16(p);
#endif
  return make_float4(k3_land(__uint_as_float(u[0])), k3_land(__uint_as_float(u[1])),
                     k3_land(__uint_as_float(u[2])), k3_land(__uint_as_float(u[3])));
}
#endif

K3_DEV float k3_unit_sq(float4 v) {
  float p = 0.0f;
  p = __builtin_fmaf(v.x, v.x, p);
  p = __builtin_fmaf(v.y, v.y, p);
  p = __builtin_fmaf(v.z, v.z, p);
  p = __builtin_fmaf(v.w, v.w, p);
  return p;
}

K3_DEV k3_u2 k3_norm4(float4 v, float sc, k3_u2 g) {
  k3_u2 o;
  o[0] = k3_mul_bf2(k3_pack_bf2(v.x * sc, v.y * sc), g[0]);
  o[1] = k3_mul_bf2(k3_pack_bf2(v.z * sc, v.w * sc), g[1]);
  return o;
}

extern "C" __global__ void __launch_bounds__(PG_THREADS) kern_k3_mla_prep_gate(
    const k3_mla_t* __restrict__ partial, uint16_t* __restrict__ mla_gate, int B) {
  const int c = PG_COLS * threadIdx.x;
  const int r0 = blockIdx.x * PG_ROWS;
  k3_u4 o[PG_ROWS];
#pragma unroll
  for (int r = 0; r < PG_ROWS; ++r) {
    const int b = min(r0 + r, B - 1);  // loads stay in bounds; stores are predicated
    const k3_mla_t* src = partial + (size_t)b * MLA_FUSED + HEADC + c;
#ifdef K3_MLA_BF16
    o[r] = k3_ld16_nt(src);  // already bf16: the landing is the identity
#else
    const k3_u4 a = k3_ld16_nt(src), d = k3_ld16_nt(src + 4);
    o[r][0] = k3_pack_bf2(__uint_as_float(a[0]), __uint_as_float(a[1]));
    o[r][1] = k3_pack_bf2(__uint_as_float(a[2]), __uint_as_float(a[3]));
    o[r][2] = k3_pack_bf2(__uint_as_float(d[0]), __uint_as_float(d[1]));
    o[r][3] = k3_pack_bf2(__uint_as_float(d[2]), __uint_as_float(d[3]));
#endif
  }
#pragma unroll
  for (int r = 0; r < PG_ROWS; ++r)
    if (r0 + r < B) k3_st16_nt(mla_gate + (size_t)(r0 + r) * INNER + c, o[r]);
}

// One row per 128-thread slice (4 rows per 512-thread workgroup).  With
// GATE the slice also lands its row's gate columns: those loads are issued
// first and their stores do not wait for the norms.
template <bool GATE>
K3_DEV void k3_mla_head_rows(const k3_mla_t* __restrict__ partial,
                             const uint16_t* __restrict__ gamma_q_a,
                             const uint16_t* __restrict__ gamma_kv_a,
                             const long long* __restrict__ slot_mapping,
                             uint16_t* __restrict__ slab, long long layer_off,
                             long long page_stride, uint16_t* __restrict__ q_norm,
                             uint16_t* __restrict__ mla_gate, int B) {
  __shared__ float red_q[PH_ROWS][12];
  __shared__ float red_k[PH_ROWS][4];
  const int row = threadIdx.x / 128;
  const int sub = (threadIdx.x / 32) % 4;  // half-wave within the row slice
  const int lane = threadIdx.x & 31;
  const int b = blockIdx.x * PH_ROWS + row;
  const bool live = b < B;
  const k3_mla_t* __restrict__ P = partial + (size_t)(live ? b : 0) * MLA_FUSED;

  constexpr int GV = INNER / 8 / 128;  // gate vectors (8 values) per thread
  k3_u4 gv[GATE ? GV : 1];
  if (GATE) {
#pragma unroll
    for (int k = 0; k < GV; ++k) {
      const k3_mla_t* src = P + HEADC + 8 * ((threadIdx.x & 127) + 128 * k);
#ifdef K3_MLA_BF16
      gv[k] = k3_ld16_nt(src);
#else
      const k3_u4 x = k3_ld16_nt(src), y = k3_ld16_nt(src + 4);
      gv[k][0] = k3_pack_bf2(__uint_as_float(x[0]), __uint_as_float(x[1]));
      gv[k][1] = k3_pack_bf2(__uint_as_float(x[2]), __uint_as_float(x[3]));
      gv[k][2] = k3_pack_bf2(__uint_as_float(y[0]), __uint_as_float(y[1]));
      gv[k][3] = k3_pack_bf2(__uint_as_float(y[2]), __uint_as_float(y[3]));
#endif
    }
  }
  float4 qv[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) qv[k] = k3_mla_ld4(P + 4 * (32 * (3 * sub + k) + lane));
  const float4 kv = k3_mla_ld4(P + 4 * (QU + 32 * sub + lane));
  // Everything the stores after the barrier need is requested now, so that
  // the slot lookup, the gammas and the rope units travel under the reductions.
  const bool rope_lane = sub == 0 && lane < ROPE / 4;
  float4 rv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (rope_lane) rv = k3_mla_ld4(P + 4 * (KU + lane));
  const long long slot = live ? slot_mapping[b] : -1;
  k3_u2 gq[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) gq[k] = *(const k3_u2*)(gamma_q_a + 4 * (32 * (3 * sub + k) + lane));
  const k3_u2 gk = *(const k3_u2*)(gamma_kv_a + 4 * (32 * sub + lane));
  if (GATE && live) {
#pragma unroll
    for (int k = 0; k < GV; ++k)
      k3_st16_nt(mla_gate + (size_t)b * INNER + 8 * ((threadIdx.x & 127) + 128 * k), gv[k]);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float p = k3_sum32(k3_unit_sq(qv[k]));
    if (lane == 0) red_q[row][3 * sub + k] = p;
  }
  {
    const float p = k3_sum32(k3_unit_sq(kv));
    if (lane == 0) red_k[row][sub] = p;
  }
  __syncthreads();
  float tq = 0.0f, tk = 0.0f;
#pragma unroll
  for (int w = 0; w < 12; ++w) tq += red_q[row][w];
#pragma unroll
  for (int w = 0; w < 4; ++w) tk += red_k[row][w];
  const float scq = k3_rsqrt_cr(__builtin_fmaf(tq, 1.0f / Q_LORA, EPSV));
  const float sck = k3_rsqrt_cr(__builtin_fmaf(tk, 1.0f / KV_LORA, EPSV));
  if (!live) return;

#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int u = 32 * (3 * sub + k) + lane;
    *(k3_u2*)(q_norm + (size_t)b * Q_LORA + 4 * u) = k3_norm4(qv[k], scq, gq[k]);
  }
  if (slot < 0) return;
  uint16_t* const rowp = slab + (slot / 64) * page_stride + layer_off + (slot % 64) * KV_A;
  *(k3_u2*)(rowp + 4 * (32 * sub + lane)) = k3_norm4(kv, sck, gk);
  if (rope_lane) {  // the row's 16 rope units: a landing only
    k3_u2 o;
    o[0] = k3_pack_bf2(rv.x, rv.y);
    o[1] = k3_pack_bf2(rv.z, rv.w);
    *(k3_u2*)(rowp + KV_LORA + 4 * lane) = o;
  }
}

extern "C" __global__ void __launch_bounds__(PH_THREADS) kern_k3_mla_prep_head(
    const k3_mla_t* __restrict__ partial, const uint16_t* __restrict__ gamma_q_a,
    const uint16_t* __restrict__ gamma_kv_a, const long long* __restrict__ slot_mapping,
    uint16_t* __restrict__ slab, long long layer_off, long long page_stride,
    uint16_t* __restrict__ q_norm, int B) {
  k3_mla_head_rows<false>(partial, gamma_q_a, gamma_kv_a, slot_mapping, slab, layer_off,
                          page_stride, q_norm, nullptr, B);
}

// Both halves in one launch (no reference counterpart: the reference launches
// head and gate separately): grid ceil(B / 4), block 512.
extern "C" __global__ void __launch_bounds__(PH_THREADS) k3h_mla_prep_fused(
    const k3_mla_t* __restrict__ partial, const uint16_t* __restrict__ gamma_q_a,
    const uint16_t* __restrict__ gamma_kv_a, const long long* __restrict__ slot_mapping,
    uint16_t* __restrict__ slab, long long layer_off, long long page_stride,
    uint16_t* __restrict__ q_norm, uint16_t* __restrict__ mla_gate, int B) {
  k3_mla_head_rows<true>(partial, gamma_q_a, gamma_kv_a, slot_mapping, slab, layer_off,
                         page_stride, q_norm, mla_gate, B);
}
