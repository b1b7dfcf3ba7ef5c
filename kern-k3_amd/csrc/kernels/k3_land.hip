// Landing kernels of the shared-expert MLP and the MoE latent norm.  One source,
// four module keys (the define K3_LAND_MODULE is implied by the base name):
//
//   k3_land (1; k3_land.cu):
//     kern_k3_rms(x, gamma, o, h, B)                 grid (B), block 1024
//     kern_k3_land(p, o, n, off, ldc, B)             grid (B, ceil(n/1024)), block 1024
//     kern_k3_land_situ(p, act, n, B)                grid (B, ceil(n/1024)), block 1024
//   k3_land_bf16 (2; k3_land_bf16.cu):
//     kern_k3_land_situ_bf16(p, act, n, B)           grid (B, ceil(n/1024)), any block
//     kern_k3_land_add2_bf16(p1, p2, prefix2, hidden, two, B)   grid (B, gy), any block
//   k3_situ_bf16 (3; k3_situ_bf16.cu):
//     kern_k3_situ_bf16(p, out, n, rows)             grid (rows, ceil(n/1024)), block 1024
//   k3_land_fused (4; k3_land_fused.cu):
//     kern_k3_situ_rms_bf16(sp, act, lat, gam, ln, n, B, h, L)
//                                                    grid 3 ceil(tokens/16), block 512
//
// Semantics (bf16 = RNE landing of an f32 value; (x) = bf16 x bf16 -> bf16):
//   rms:   r = 1 / sqrt(sum_i x_i^2 / h + 1e-5);  o_i = bf16(x_i * r) (x) gamma_i
//          (k3_land.cu:21-25, 104-165).  The sum replays the reference's order:
//          1024 "threads" tid, each summing its 16-byte vectors u = tid + 1024 r
//          (8 fma steps per vector), a 32-lane xor butterfly per warp of 32 tids,
//          then a 32-lane butterfly over the 32 warp partials.
//   land:  o[b, i] = bf16(p[b * ldc + off + i])  (k3_land.cu:27, 168-190).
//   situ:  g = bf16(p[b, i]), u = bf16(p[b, n + i]) (gate | up halves of a row of
//          2n), act[b, i] = bf16((4 tanh(g/4) * sigmoid(g)) * (25 tanh(u * 0.04)))
//          (k3_land.cu:29-34, 200-237; k3_land_bf16.cu:1-20; k3_situ_bf16.cu).
//   add2:  hidden = bf16(f32(prefix2) + f32(p1) [+ f32(p2)]), left to right
//          (k3_land_bf16.cu:84-140).
//   situ_rms: blockIdx % 3 == 0 -> rms rows [4q, 4q + 4) of lat (h wide, < L,
//          only the first 512 vectors of a row, as the reference's one-vector-per-
//          thread job; nothing when h % 8 != 0); otherwise situ rows
//          [2j, 2j + 2), j = 2q + blockIdx % 3 - 1, of sp (< B), bf16 operands
//          (k3_land_fused.cu:1-33, 151-202).
//
// Work split.  Every elementwise kernel ignores the reference's per-row mapping
// and walks the flattened [rows, n] output instead: workgroup L (the linear
// block id) owns 8 consecutive values per thread (land: two groups of 4), i.e.
// elements [L * 8 * blockDim, (L + 1) * 8 * blockDim); ids past the end exit.
// Any grid that covers the tensor works: the manifests' grids (one thread per
// value, 1024-thread blocks) do, and so do the compact grids the typed k3h
// calls launch (256-thread blocks, exactly as many as there is work) -- on
// MI355X the empty waves of the manifest grid cost more than the work (the
// (4096, 33) x 1024 grid of land_situ_n33792 takes 116 us to dispatch with no
// work at all).  The rms kernels give each wave one row (blockDim / 64 rows
// per workgroup, 4 per 512-thread rms job), lane l playing the reference
// threads l + 64 k of its 1024-thread block, so no workgroup barrier is
// needed; shapes outside that fast path (h % 8 != 0 or h > 8192) run the
// reference's own layout, one row per workgroup of blockDim (1024) threads.
//
// SiTU numerics: tanh and the logistic are evaluated from the hardware 2^x and
// reciprocal (v_exp_f32, v_rcp_f32), with an odd Taylor series near 0 where
// 1 - e^-2x would cancel; every output is within one bf16 ulp of the exact
// value of the formula (the reference's tanh.approx / __expf / __frcp_rn form
// is pinned to the same tolerance).
#include "../common/k3_dev.h"
#include "k3_situ.h"

#ifndef K3_LAND_MODULE
#define K3_LAND_MODULE 1
#endif

#define K3_RMS_EPS 1e-5f
// Eight bf16 gate values and eight bf16 up values -> eight bf16 outputs.  The
// landing kernels take the branch form of the SiTU math (k3_situ<false>).
K3_DEV k3_u4 k3_situ8(k3_u4 g, k3_u4 u) {
  k3_u4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = k3_pack_bf2(k3_situ<false>(k3_bf_lo(g[j]), k3_bf_lo(u[j])),
                       k3_situ<false>(k3_bf_hi(g[j]), k3_bf_hi(u[j])));
  return o;
}

// Eight f32 -> eight bf16 (two 16-byte loads' worth).
K3_DEV k3_u4 k3_land8(k3_u4 a, k3_u4 b) {
  k3_u4 o;
  o[0] = k3_pack_bf2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  o[1] = k3_pack_bf2(__uint_as_float(a[2]), __uint_as_float(a[3]));
  o[2] = k3_pack_bf2(__uint_as_float(b[0]), __uint_as_float(b[1]));
  o[3] = k3_pack_bf2(__uint_as_float(b[2]), __uint_as_float(b[3]));
  return o;
}

K3_DEV uint32_t k3_linear_block() {
  return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}

// ---------------------------------------------------------------- rms rows
// Lane-0 value of a 32-lane xor butterfly (offsets 16 .. 1) over w[0..31] with
// w[i] = 0 for i >= nw (every lane of the butterfly ends with these bits).
K3_DEV float k3_bfly32_tree(const float* w, int nw) {
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = (i < nw ? w[i] : 0.0f) + (i + 16 < nw ? w[i + 16] : 0.0f);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) {
#pragma unroll
    for (int i = 0; i < o; ++i) a[i] = a[i] + a[i + o];
  }
  return a[0];
}

// One row of the rms on one wave: lane l plays reference threads l + 64 k
// (k < NK), each with the single vector u = l + 64 k < nvec (the reference
// threads' only vector when the row has at most 1024 / 512 of them).  The
// warp of reference threads 32 m .. 32 m + 31 is the half-wave (m & 1) at
// slot k = m / 2.
template <int NK>
K3_DEV void k3_rms_row_wave(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ gamma,
                            uint16_t* __restrict__ orow, int nvec, int h, int lane) {
  // NK <= 8: every load (the row, then gamma) is issued before the reduction, so
  // that no load waits behind a store (the vector memory counter retires in
  // order); wider rows load gamma beside the stores (register budget)
  constexpr bool PRE = NK <= 8;
  k3_u4 xv[NK], gv[PRE ? NK : 1];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (k * 64 >= nvec) break;
    const int u = min(lane + 64 * k, nvec - 1);
    xv[k] = k3_ld16_nt(xr + 8 * u);
  }
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      if (k * 64 >= nvec) break;
      const int u = min(lane + 64 * k, nvec - 1);
      gv[k] = k3_ld16(gamma + 8 * u);
    }
  }
  float wsum[2 * NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (k * 64 >= nvec) { wsum[2 * k] = 0.0f; wsum[2 * k + 1] = 0.0f; continue; }
    float s = 0.0f;
    if (lane + 64 * k < nvec) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = k3_bf_lo(xv[k][j]), hi = k3_bf_hi(xv[k][j]);
        s = __builtin_fmaf(lo, lo, s);
        s = __builtin_fmaf(hi, hi, s);
      }
    }
    s = k3_sum32(s);
    wsum[2 * k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
    wsum[2 * k + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
  }
  const float tot = k3_bfly32_tree(wsum, 2 * NK);
  const float r = k3_rsqrt_cr(tot / (float)h + K3_RMS_EPS);
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (k * 64 >= nvec) break;
    const int u = lane + 64 * k;
    if (u < nvec) {
      const k3_u4 g = PRE ? gv[PRE ? k : 0] : k3_ld16(gamma + 8 * u);
      k3_u4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(xv[k][j]) * r, k3_bf_hi(xv[k][j]) * r), g[j]);
      k3_st16_nt(orow + 8 * u, o);
    }
  }
}

#if K3_LAND_MODULE == 1
// Reference layout for shapes outside the one-wave path: one row per 1024-thread
// workgroup, thread tid sums its vectors u = tid + 1024 r (or, for h % 8 != 0,
// its elements i = tid + 1024 r), warp butterflies, then a butterfly over the
// 32 warp partials (k3_land.cu:112-165).
K3_DEV void k3_rms_row_block(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ gamma,
                             uint16_t* __restrict__ orow, int h) {
  __shared__ float s_w[32];
  const int tid = threadIdx.x;
  const bool vec = (h & 7) == 0;
  float s = 0.0f;
  const int nt = (int)blockDim.x;  // 1024 in the manifest, the order the checker replays
  if (vec) {
    for (int u = tid; u < (h >> 3); u += nt) {
      const k3_u4 x = k3_ld16(xr + 8 * u);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = k3_bf_lo(x[j]), hi = k3_bf_hi(x[j]);
        s = __builtin_fmaf(lo, lo, s);
        s = __builtin_fmaf(hi, hi, s);
      }
    }
  } else {
    for (int i = tid; i < h; i += nt) {
      const float v = k3_bf(xr[i]);
      s = __builtin_fmaf(v, v, s);
    }
  }
  s = k3_sum32(s);
  if ((tid & 31) == 0) s_w[tid >> 5] = s;
  __syncthreads();
  const int nw = (int)(blockDim.x >> 5);  // warps of the block; the rest count as 0
  float w[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) w[i] = i < nw ? s_w[i] : 0.0f;
  const float r = k3_rsqrt_cr(k3_bfly32_tree(w, nw) / (float)h + K3_RMS_EPS);
  if (vec) {
    for (int u = tid; u < (h >> 3); u += nt) {
      const k3_u4 x = k3_ld16(xr + 8 * u);
      const k3_u4 g = k3_ld16(gamma + 8 * u);
      k3_u4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = k3_mul_bf2(k3_pack_bf2(k3_bf_lo(x[j]) * r, k3_bf_hi(x[j]) * r), g[j]);
      k3_st16(orow + 8 * u, o);
    }
  } else {
    for (int i = tid; i < h; i += nt) {
      const uint32_t y = k3_pack_bf2(k3_bf(xr[i]) * r, 0.0f);
      orow[i] = (uint16_t)k3_mul_bf2(y, gamma[i]);
    }
  }
}

extern "C" __global__ void __launch_bounds__(1024) kern_k3_rms(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, uint16_t* __restrict__ o,
    int h, int B) {
  if (h <= 0) return;
  if ((h & 7) == 0 && h <= 8192) {
    // one row per wave (16 per 1024-thread workgroup); the sum replays the
    // reference's 1024-thread block, the launch geometry of the manifest
    const int b = blockIdx.x * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
    if (b >= B) return;
    const int nvec = h >> 3;
    if (nvec <= 512)  // h <= 4096: up to 8 vectors per lane
      k3_rms_row_wave<8>(x + (size_t)b * h, gamma, o + (size_t)b * h, nvec, h, threadIdx.x & 63);
    else
      k3_rms_row_wave<16>(x + (size_t)b * h, gamma, o + (size_t)b * h, nvec, h, threadIdx.x & 63);
    return;
  }
  const int b = blockIdx.x;
  if (b >= B) return;
  k3_rms_row_block(x + (size_t)b * h, gamma, o + (size_t)b * h, h);
}

extern "C" __global__ void __launch_bounds__(1024) kern_k3_land(
    const float* __restrict__ p, uint16_t* __restrict__ o, int n, int off, int ldc, int B) {
  if (n <= 0 || B <= 0) return;
  const long long total = (long long)B * n;
  if (((n | off | ldc) & 3) == 0) {
    // two 4-value groups per thread over the flattened [B, n] output, group k of
    // the workgroup's 2 * blockDim at k * blockDim + tid (coalesced per k)
    const long long q0 = (long long)k3_linear_block() * 2 * blockDim.x + threadIdx.x;
    const int nq = n >> 2;
    k3_u4 a[2];
    long long e[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      e[k] = q0 + (long long)k * blockDim.x;
      const long long q = min(e[k], total / 4 - 1);
      const long long row = q / nq, c = (q - row * nq) * 4;
      a[k] = k3_ld16_nt(p + row * ldc + off + c);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (e[k] * 4 >= total) break;
      k3_u2 w;
      w[0] = k3_pack_bf2(__uint_as_float(a[k][0]), __uint_as_float(a[k][1]));
      w[1] = k3_pack_bf2(__uint_as_float(a[k][2]), __uint_as_float(a[k][3]));
      k3_st8_nt(o + e[k] * 4, w);
    }
    return;
  }
  const int b = blockIdx.x;
  if (b >= B) return;
  for (int i = blockIdx.y * blockDim.x + threadIdx.x; i < n; i += gridDim.y * blockDim.x)
    o[(size_t)b * n + i] = (uint16_t)k3_pack_bf2(p[(size_t)b * ldc + off + i], 0.0f);
}

extern "C" __global__ void __launch_bounds__(1024) kern_k3_land_situ(
    const float* __restrict__ p, uint16_t* __restrict__ act, int n, int B) {
  if (n <= 0 || B <= 0) return;
  if ((n & 7) == 0) {
    // 8 consecutive outputs per thread over the flattened [B, n] output
    const long long total = (long long)B * n;
    const long long e = ((long long)k3_linear_block() * blockDim.x + threadIdx.x) * 8;
    if (e >= total) return;
    const long long row = e / n, c = e - row * n;
    const float* pg = p + row * 2 * n + c;
    const k3_u4 g0 = k3_ld16_nt(pg), g1 = k3_ld16_nt(pg + 4);
    const k3_u4 u0 = k3_ld16_nt(pg + n), u1 = k3_ld16_nt(pg + n + 4);
    // both operands land to bf16 first (k3_land.cu:200-204)
    k3_st16_nt(act + e, k3_situ8(k3_land8(g0, g1), k3_land8(u0, u1)));
    return;
  }
  const int b = blockIdx.x;
  if (b >= B) return;
  for (int i = blockIdx.y * blockDim.x + threadIdx.x; i < n; i += gridDim.y * blockDim.x) {
    const float g = k3_land(p[(size_t)b * 2 * n + i]);
    const float u = k3_land(p[(size_t)b * 2 * n + n + i]);
    act[(size_t)b * n + i] = (uint16_t)k3_pack_bf2(k3_situ<false>(g, u), 0.0f);
  }
}
#endif  // K3_LAND_MODULE == 1

#if K3_LAND_MODULE == 2 || K3_LAND_MODULE == 3
// bf16 gate | up rows of 2n -> act [rows, n]; see kern_k3_land_situ.
K3_DEV void k3_situ_bf16_body(const uint16_t* __restrict__ p, uint16_t* __restrict__ act, int n,
                              int rows) {
  if (n <= 0 || rows <= 0) return;
  if ((n & 7) == 0) {
    const long long total = (long long)rows * n;
    const long long e = ((long long)k3_linear_block() * blockDim.x + threadIdx.x) * 8;
    if (e >= total) return;
    const long long row = e / n, c = e - row * n;
    const uint16_t* pg = p + row * 2 * n + c;
    const k3_u4 g = k3_ld16_nt(pg), u = k3_ld16_nt(pg + n);
    k3_st16_nt(act + e, k3_situ8(g, u));
    return;
  }
  const int b = blockIdx.x;
  if (b >= rows) return;
  for (int i = blockIdx.y * blockDim.x + threadIdx.x; i < n; i += gridDim.y * blockDim.x)
    act[(size_t)b * n + i] = (uint16_t)k3_pack_bf2(
        k3_situ<false>(k3_bf(p[(size_t)b * 2 * n + i]), k3_bf(p[(size_t)b * 2 * n + n + i])), 0.0f);
}
#endif

#if K3_LAND_MODULE == 2
extern "C" __global__ void __launch_bounds__(1024) kern_k3_land_situ_bf16(
    const uint16_t* __restrict__ p, uint16_t* __restrict__ act, int n, int B) {
  k3_situ_bf16_body(p, act, n, B);
}

// hidden = bf16(f32(prefix2) + f32(p1) [+ f32(p2)]): row blockIdx.x, vectors
// blockIdx.y * blockDim + tid, stride gridDim.y * blockDim (any geometry that
// covers the row, as the reference's k3_land_bf16.cu:96-140).
extern "C" __global__ void __launch_bounds__(1024) kern_k3_land_add2_bf16(
    const uint16_t* __restrict__ p1, const uint16_t* __restrict__ p2,
    const uint16_t* __restrict__ prefix2, uint16_t* __restrict__ hidden, int two, int B) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const size_t row = (size_t)b * 7168;
  for (int v = blockIdx.y * blockDim.x + threadIdx.x; v < 896; v += gridDim.y * blockDim.x) {
    const size_t off = row + 8 * v;
    const k3_u4 a = k3_ld16_nt(p1 + off);
    const k3_u4 c = k3_ld16_nt(prefix2 + off);
    k3_u4 e = {0u, 0u, 0u, 0u};
    if (two) e = k3_ld16_nt(p2 + off);
    k3_u4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x = k3_bf_lo(c[j]) + k3_bf_lo(a[j]);
      float y = k3_bf_hi(c[j]) + k3_bf_hi(a[j]);
      if (two) {
        x += k3_bf_lo(e[j]);
        y += k3_bf_hi(e[j]);
      }
      o[j] = k3_pack_bf2(x, y);
    }
    k3_st16_nt(hidden + off, o);
  }
}
#endif  // K3_LAND_MODULE == 2

#if K3_LAND_MODULE == 3
extern "C" __global__ void __launch_bounds__(1024) kern_k3_situ_bf16(
    const uint16_t* __restrict__ p, uint16_t* __restrict__ out, int n, int rows) {
  k3_situ_bf16_body(p, out, n, rows);
}
#endif  // K3_LAND_MODULE == 3

#if K3_LAND_MODULE == 4
// Job layout of the reference (k3_land_fused.cu:151-156): of every three
// consecutive workgroups the first normalises 4 latent rows, the other two
// land 2 SiTU rows each.
extern "C" __global__ void __launch_bounds__(512) kern_k3_situ_rms_bf16(
    const uint16_t* __restrict__ sp, uint16_t* __restrict__ act, const uint16_t* __restrict__ lat,
    const uint16_t* __restrict__ gam, uint16_t* __restrict__ ln, int n, int B, int h, int L) {
  const int q = blockIdx.x / 3;
  const int job = blockIdx.x - 3 * q;
  const int tid = threadIdx.x;
  if (job == 0) {
    // the reference's rms job: one 16-byte vector per thread of 512, rows < L,
    // nothing stored when h % 8 != 0
    if ((h & 7) != 0 || h <= 0) return;
    const int w = tid >> 6;
    const int row = 4 * q + w;
    if (w >= 4 || row >= L) return;
    const int nvec = min(h >> 3, 512);
    k3_rms_row_wave<8>(lat + (size_t)row * h, gam, ln + (size_t)row * h, nvec, h, tid & 63);
    return;
  }
  const int j0 = 2 * q + (job - 1);
  if (n <= 0) return;
  if ((n & 7) == 0) {
    // the two rows' 2 n / 8 output vectors, three loads in flight per thread
    const int nv = n >> 3;
    const int rows = min(2, B - 2 * j0);
    if (rows <= 0) return;
    const int tot = rows * nv;
    for (int k0 = tid; k0 < tot; k0 += 3 * 512) {
      k3_u4 g[3], u[3];
#pragma unroll
      for (int s = 0; s < 3; ++s) {
        const int k = min(k0 + s * 512, tot - 1);
        const int r = k / nv, c = k - r * nv;
        const uint16_t* pg = sp + (size_t)(2 * j0 + r) * 2 * n + 8 * c;
        g[s] = k3_ld16_nt(pg);
        u[s] = k3_ld16_nt(pg + n);
      }
#pragma unroll
      for (int s = 0; s < 3; ++s) {
        const int k = k0 + s * 512;
        if (k >= tot) break;
        const int r = k / nv, c = k - r * nv;
        k3_st16_nt(act + (size_t)(2 * j0 + r) * n + 8 * c, k3_situ8(g[s], u[s]));
      }
    }
    return;
  }
  for (int r = 0; r < 2; ++r) {
    const int row = 2 * j0 + r;
    if (row >= B) break;
    for (int i = tid; i < n; i += 512)
      act[(size_t)row * n + i] = (uint16_t)k3_pack_bf2(
          k3_situ<false>(k3_bf(sp[(size_t)row * 2 * n + i]), k3_bf(sp[(size_t)row * 2 * n + n + i])),
          0.0f);
  }
}
#endif  // K3_LAND_MODULE == 4
