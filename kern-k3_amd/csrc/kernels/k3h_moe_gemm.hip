// Module k3h_moe_gemm: the MoE expert GEMMs on the MX-scaled matrix cores
// (v_mfma_scale_f32_32x32x64_f8f6f4), in place of the reference's prebuilt
// batched GEMMs moe_fc1 / moe_fc2 (manifest ops moe_fc1, moe_fc2; MxE4m3
// activations x MxE2m1 weights, f32 accumulation; kernels.toml:1-9).
//
//   C[r, n] = sum_k a(r, k) * w_e(n, k),  e = cta_batch[r / 128]
//   a(r, k) = e4m3(a_q[src(r), k]) * 2^(a_sf[src(r), k / 32] - 127)
//   w_e(n, k) = e2m1(w[e, n, k]) * 2^(w_sf[e, n, k / 32] - 127)
//   src(r) = a_rows ? a_rows[r] : r   (a_rows = route_map: fc1 gathers its rows
//            from the token-ordered activations as the reference's fc1 does;
//            null reads rows already permuted by kern_k3_moe_permute_mx)
//
// over the 128-row route tiles t < *num_tiles of the routing tables
// (kern_k3_moe_route_tables), rows [128 t, 128 t + 128).  Epilogues:
//   kern_k3h_moe_gemm_f32       out f32 [rows, N]            (the raw accumulators)
//   kern_k3h_moe_gemm_bf16      out bf16 [rows, N]           (fc2: bf16(C))
//   kern_k3h_moe_gemm_situ_mx   out e4m3 [rows, N / 2] + E8M0 [rows, N / 64]
//       (fc1: the weight rows are [up; gate] halves of N / 2 each; with
//        u = bf16(C[r, j]), g = bf16(C[r, N / 2 + j]) the activation
//        x = bf16(situ(g, u; alpha[e], beta[e])) is quantised per 32 columns
//        exactly as kern_k3_moe_quant quantises a bf16 row)
//
// Weight layouts (built once at load time by kern_k3h_moe_w_tile /
// kern_k3h_moe_sf_tile from the row-major [E, N, K / 2] e2m1 (low nibble = even
// k) and [E, N, K / 32] E8M0 tensors, in place of kern_k3_moe_w_shuffle /
// kern_k3_moe_sf_shuffle):
//   wt  [E][N / 32][K / 64][64][16 B]: lane l = (j = l % 32, h = l / 32) of the
//       32-column tile T holds row R(T, j), k in [64 kt + 32 h, + 32) -- exactly
//       the B operand of one MFMA, so each operand is one 1 KB coalesced load;
//   wsf [E][N / 32][K / 128][64][2 B]: byte s = scale block 4 ks + 2 s + h of R(T, j).
//   R(T, j) = 32 T + j, or for the gated fc1 weights (tile order up, gate, up,
//   gate, ...) R(2 t, j) = 32 t + j (up) and R(2 t + 1, j) = N / 2 + 32 t + j (gate),
//   so a wave holds an up tile and its gate tile in the same accumulator lanes.
//
// MFMA operand layouts (gfx950, measured): the e4m3 A operand of lane
// (i = l % 32, h = l / 32) holds row i at k = 16 h + p (byte p < 16) and
// k = 32 + 16 h + p - 16 (p >= 16); the e2m1 B operand holds column j at
// k = 32 h + p (nibble p of dwords 0-3); each lane's scale byte covers its
// row / column over the 32-block h; accumulator VGPR q of lane l is
// C[8 (q / 4) + 4 h + q % 4, l % 32].
//
// Work split: workgroup (x, t) = 256 logical columns x route tile t; 4 waves,
// wave w owns rows 64 (w / 2) .. + 64 and columns 128 (w % 2) .. + 128 (2 x 4
// MFMA tiles, 128 accumulator registers); K steps of 128, the next step's
// operands loaded while this step's 16 MFMAs run.  Consecutive x of a tile land
// on consecutive XCDs (round-robin dispatch), and with N / 256 a multiple of 8
// every tile's column block x stays on XCD x % 8, so each XCD's L2 holds one
// eighth of every expert's weights.
#include "../common/k3_dev.h"
#include "k3_situ.h"

typedef int k3_v8i __attribute__((ext_vector_type(8)));
typedef float k3_v16f __attribute__((ext_vector_type(16)));

#define K3G_TILE_M 128
#define K3G_TILE_N 256
#define K3G_KSTEP 128

// ---------------------------------------------------------------- layouts
K3_DEV int k3g_row(int T, int j, int n, int gated) {
  if (!gated) return 32 * T + j;
  return (T & 1 ? n / 2 : 0) + 32 * (T >> 1) + j;
}

// One thread per 16-byte operand slice: slice id = ((e * NT + T) * KT + kt) * 64 + l.
extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_w_tile(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int experts, int n, int k,
    int gated) {
  const long long NT = n / 32, KT = k / 64;
  const long long total = (long long)experts * NT * KT * 64;
  const long long rb = k / 2;
  for (long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (long long)gridDim.x * blockDim.x) {
    const int l = (int)(id & 63);
    const long long q = id >> 6;
    const int kt = (int)(q % KT);
    const long long et = q / KT;
    const int T = (int)(et % NT);
    const long long e = et / NT;
    const int r = k3g_row(T, l & 31, n, gated);
    const uint8_t* s = src + (e * n + r) * rb + 32 * kt + 16 * (l >> 5);
    k3_st16(dst + id * 16, k3_ld16(s));
  }
}

// One thread per (e, T, ks, l): two scale bytes.
extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_sf_tile(
    const uint8_t* __restrict__ src, uint16_t* __restrict__ dst, int experts, int n, int k,
    int gated) {
  const long long NT = n / 32, KS = k / 128, KG = k / 32;
  const long long total = (long long)experts * NT * KS * 64;
  for (long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (long long)gridDim.x * blockDim.x) {
    const int l = (int)(id & 63);
    const long long q = id >> 6;
    const int ks = (int)(q % KS);
    const long long et = q / KS;
    const int T = (int)(et % NT);
    const long long e = et / NT;
    const int r = k3g_row(T, l & 31, n, gated);
    const uint8_t* s = src + (e * n + r) * KG + 4 * ks + (l >> 5);
    dst[id] = (uint16_t)(s[0] | (s[2] << 8));
  }
}

// ---------------------------------------------------------------- main loop
struct K3gStep {
  k3_u4 alo[2][2], ahi[2][2];  // [m tile][substep]
  uint32_t sa[2];              // A scale bytes of blocks 4 ks .. 4 ks + 3
  k3_u4 b[4][2];               // [n tile][substep]
  uint32_t sb[4];              // B scale bytes (substep 0 | substep 1 << 8)
};

K3_DEV void k3g_load(K3gStep& st, const uint8_t* const* ap, const uint8_t* const* sp,
                     const uint8_t* const* wp, const uint16_t* const* wsp, int ks, int h) {
  const int k0 = ks * K3G_KSTEP;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      st.alo[mt][s] = k3_ld16(ap[mt] + k0 + 64 * s + 16 * h);
      st.ahi[mt][s] = k3_ld16(ap[mt] + k0 + 64 * s + 32 + 16 * h);
    }
    st.sa[mt] = *(const uint32_t*)(sp[mt] + k0 / 32);
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
    for (int s = 0; s < 2; ++s) st.b[nt][s] = k3_ld16(wp[nt] + (size_t)(2 * ks + s) * 1024);
    st.sb[nt] = wsp[nt][(size_t)ks * 64];
  }
}

K3_DEV void k3g_mma(k3_v16f (&acc)[2][4], const K3gStep& st, int h) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const k3_u4 lo = st.alo[mt][s], hi = st.ahi[mt][s];
      const k3_v8i a = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                        (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      const int sa = (int)(st.sa[mt] >> (16 * s + 8 * h));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const k3_u4 bv = st.b[nt][s];
        const k3_v8i b = {(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3], 0, 0, 0, 0};
        const int sb = (int)(st.sb[nt] >> (8 * s));
        acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[mt][nt], 0, 4, 0,
                                                                       sa, 0, sb);
      }
    }
  }
}

// Accumulates the wave's 64 x 128 block; returns false when the tile is past
// the routing tables' live count or its expert is out of range (the whole
// workgroup exits).
K3_DEV bool k3g_block(k3_v16f (&acc)[2][4], const uint8_t* __restrict__ a,
                      const uint8_t* __restrict__ a_sf, const int* __restrict__ a_rows,
                      const uint8_t* __restrict__ wt, const uint16_t* __restrict__ wsf,
                      const int* __restrict__ num_tiles, const int* __restrict__ cta_batch, int E,
                      int N, int K, int& tile, int& e, int& lane, int& wm, int& wn) {
  tile = blockIdx.y;
  if (tile >= *num_tiles) return false;
  e = cta_batch[tile];
  if (e < 0 || e >= E) return false;
  const int w = threadIdx.x >> 6;
  lane = threadIdx.x & 63;
  wm = w >> 1;
  wn = w & 1;
  const int h = lane >> 5, j = lane & 31;
  const int KG = K / 32, KT = K / 64, KS = K / K3G_KSTEP, NT = N / 32;

  const uint8_t* ap[2];
  const uint8_t* sp[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int r = tile * K3G_TILE_M + 64 * wm + 32 * mt + j;
    int src = a_rows ? a_rows[r] : r;
    src = src < 0 ? 0 : src;
    ap[mt] = a + (size_t)src * K;
    sp[mt] = a_sf + (size_t)src * KG;
  }
  const uint8_t* wp[4];
  const uint16_t* wsp[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int T = blockIdx.x * (K3G_TILE_N / 32) + 4 * wn + nt;
    wp[nt] = wt + ((size_t)e * NT + T) * KT * 1024 + lane * 16;
    wsp[nt] = wsf + ((size_t)e * NT + T) * KS * 64 + lane;
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[mt][nt][q] = 0.0f;

  K3gStep cur, nxt;
  k3g_load(cur, ap, sp, wp, wsp, 0, h);
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + 1 < KS) k3g_load(nxt, ap, sp, wp, wsp, ks + 1, h);
    k3g_mma(acc, cur, h);
    cur = nxt;
  }
  return true;
}

// Row of accumulator register q of m tile mt, within the route tile.
K3_DEV int k3g_out_row(int wm, int mt, int q, int h) {
  return 64 * wm + 32 * mt + 8 * (q >> 2) + 4 * h + (q & 3);
}

#define K3G_PARAMS                                                                          \
  const uint8_t *__restrict__ a, const uint8_t *__restrict__ a_sf,                          \
      const int *__restrict__ a_rows, const uint8_t *__restrict__ wt,                       \
      const uint16_t *__restrict__ wsf, const int *__restrict__ num_tiles,                  \
      const int *__restrict__ cta_batch, int E, int N, int K

extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_gemm_f32(K3G_PARAMS,
                                                                        float* __restrict__ out) {
  k3_v16f acc[2][4];
  int tile, e, lane, wm, wn;
  if (!k3g_block(acc, a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, tile, e, lane, wm, wn))
    return;
  const int h = lane >> 5, j = lane & 31;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = blockIdx.x * K3G_TILE_N + 128 * wn + 32 * nt + j;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const size_t row = (size_t)tile * K3G_TILE_M + k3g_out_row(wm, mt, q, h);
        out[row * N + col] = acc[mt][nt][q];
      }
    }
}

extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_gemm_bf16(K3G_PARAMS,
                                                                         uint16_t* __restrict__ out) {
  k3_v16f acc[2][4];
  int tile, e, lane, wm, wn;
  if (!k3g_block(acc, a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, tile, e, lane, wm, wn))
    return;
  const int h = lane >> 5, j = lane & 31;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = blockIdx.x * K3G_TILE_N + 128 * wn + 32 * nt + j;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const size_t row = (size_t)tile * K3G_TILE_M + k3g_out_row(wm, mt, q, h);
        out[row * N + col] = (uint16_t)k3_pack_bf2(acc[mt][nt][q], 0.0f);
      }
    }
}

// One bf16 value scaled by 2^-e to e4m3 (byte), as k3_vec_to_e4m3 does per element.
K3_DEV uint32_t k3g_to_e4m3(uint32_t xb16, int e) {
  const float f = __builtin_ldexpf(k3_bf((uint16_t)xb16), -e);
  uint32_t q = k3_pack_e4m3x2(f, 0.0f) & 0xffu;
  if (e == 127 && __builtin_isinf(f)) q = 0x7eu | (f < 0.0f ? 0x80u : 0u);
  return q;
}

// Largest value over the 32 lanes of this half-wave (ds_swizzle xor butterfly).
K3_DEV uint32_t k3g_max32_u32(uint32_t v) {
  uint32_t o = k3_swz_xor_u32<16>(v); v = v > o ? v : o;
  o = k3_swz_xor_u32<8>(v); v = v > o ? v : o;
  o = k3_swz_xor_u32<4>(v); v = v > o ? v : o;
  o = k3_swz_xor_u32<2>(v); v = v > o ? v : o;
  o = k3_swz_xor_u32<1>(v); v = v > o ? v : o;
  return v;
}

extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_gemm_situ_mx(
    K3G_PARAMS, uint8_t* __restrict__ out_q, uint8_t* __restrict__ out_sf,
    const float* __restrict__ alpha, const float* __restrict__ beta) {
  k3_v16f acc[2][4];
  int tile, e, lane, wm, wn;
  if (!k3g_block(acc, a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, tile, e, lane, wm, wn))
    return;
  const int h = lane >> 5, j = lane & 31;
  const float al = alpha[e], be = beta[e];
  const float ial = 1.0f / al, ibe = 1.0f / be;
  const int NA = N / 2;  // activation columns
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // logical tiles 2 t (up) and 2 t + 1 (gate): activation block t
      const int t = blockIdx.x * (K3G_TILE_N / 64) + 2 * wn + p;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const float u = k3_land(acc[mt][2 * p][q]);
        const float g = k3_land(acc[mt][2 * p + 1][q]);
        const uint32_t xb = k3_pack_bf2(k3_situ_gate_a(g, al, ial) * k3_situ_up_b(u, be, ibe), 0.0f);
        const int ex = k3_e8m0_exp(k3g_max32_u32(k3_absbits_nonan(xb & 0xffffu)));
        const uint32_t qb = k3g_to_e4m3(xb, ex);
        const size_t row = (size_t)tile * K3G_TILE_M + k3g_out_row(wm, mt, q, h);
        out_q[row * NA + 32 * t + j] = (uint8_t)qb;
        if (j == 0) out_sf[row * (NA / 32) + t] = (uint8_t)(ex + 127);
      }
    }
}
