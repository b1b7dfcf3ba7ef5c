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
//   wsf [E][N / 128][K / 128][64][4][2 B]: for the 4 consecutive column tiles
//       T = 4 G + u of group G, byte s of entry (ks, lane l, u) = scale block
//       4 ks + 2 s + h of R(T, j) -- a wave's 4 tiles' scales of one K step are
//       one 8-byte load per lane.
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
// MFMA tiles, 128 accumulators).  K steps of 128: the workgroup's A rows, B
// tiles and scales of a step are brought into LDS by direct-to-LDS loads one
// step ahead of the MFMAs (two stages; two workgroups per CU).  The epilogues
// pass the accumulators through LDS so that each lane owns whole output rows
// (16-byte stores; the fc1 MX blocks quantised in registers).  The workgroup's
// linear id picks its item from its XCD's share (k3g_item below), so that each
// XCD's L2 serves a fixed part of the live tiles and of the column blocks.
#include "../common/k3_dev.h"
#include <type_traits>

#include "k3_mx.h"
#include "k3_situ.h"

typedef int k3_v8i __attribute__((ext_vector_type(8)));
typedef float k3_v16f __attribute__((ext_vector_type(16)));

#define K3G_TILE_M 128
#define K3G_TILE_N 256
#define K3G_KSTEP 128
// instruction classes of __builtin_amdgcn_sched_group_barrier
#define K3G_SG_MFMA 0x008
#define K3G_SG_VMEM 0x010
#define K3G_SG_VMEM_READ 0x020
#define K3G_SG_DS_READ 0x100
#define K3G_XCDS 8  // workgroups are dispatched round-robin over the XCDs

// Exchange between the half-waves: x keeps lanes 0-31 and takes y's lanes 0-31
// into lanes 32-63; y keeps lanes 32-63 and takes x's lanes 32-63 into lanes
// 0-31 (v_permlane32_swap x, y).
K3_DEV void k3g_swap(uint32_t& x, uint32_t& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}

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

// One thread per (e, G, ks, l, u): two scale bytes (u fastest).
extern "C" __global__ void __launch_bounds__(256) kern_k3h_moe_sf_tile(
    const uint8_t* __restrict__ src, uint16_t* __restrict__ dst, int experts, int n, int k,
    int gated) {
  const long long NG = n / 128, KS = k / 128, KG = k / 32;
  const long long total = (long long)experts * NG * KS * 64 * 4;
  for (long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (long long)gridDim.x * blockDim.x) {
    const int u = (int)(id & 3);
    long long q = id >> 2;
    const int l = (int)(q & 63);
    q >>= 6;
    const int ks = (int)(q % KS);
    q /= KS;
    const int G = (int)(q % NG);
    const long long e = q / NG;
    const int r = k3g_row(4 * G + u, l & 31, n, gated);
    const uint8_t* s = src + (e * n + r) * KG + 4 * ks + (l >> 5);
    dst[id] = (uint16_t)(s[0] | (s[2] << 8));
  }
}

// ---------------------------------------------------------------- LDS pipeline
// Workgroup-shared operand stages filled by direct-to-LDS loads
// (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l).  A stage
// (one K step of 128):
//   A  16 KB: the 128 rows' 128-byte slices, swizzled (k3g_aslot); each load
//             instruction moves 8 whole row slices (measured: loading the same
//             bytes as 32 rows x 32 bytes per instruction, in MFMA operand order,
//             cost a third of the kernel's time);
//   B  16 KB: block (T * 2 + s), T = 32-column tile of the workgroup (a copy of
//             the tiled weights' 1 KB operand);
// Each wave issues 8 loads per stage (its 32 rows' A slices in 4, 4 B blocks).
// Two stages: the loads of step ks + 2 go out behind the barrier in the middle
// of step ks and must land by the middle of step ks + 1.  B scales go straight
// to registers: a wave's 4 tiles' pairs of a step, one 8-byte load per lane,
// two steps ahead (measured: as a per-stage direct-to-LDS load they cost fc1
// 7%).  The tile's A scales for the whole of K (128 rows x K/32 bytes) are
// loaded once, before the first stage, into a table behind the stages
// (measured: one 4-byte load per row and step, 32 gathered rows per
// instruction, cost fc1 15%).  The table holds KGM bytes per row at a row
// stride of KGM + 4 bytes (an odd number of dwords, so the 32 rows a wave reads
// hit 32 different banks; at 112 bytes rows r and r + 16 shared one): entries
// for K <= 3584 (KGM 112) keep two workgroups per CU (2 x 79 KB of LDS); the "_w"
// entries (KGM 224) take K <= 7168.  Two stages and at most 256 registers per
// wave let two workgroups share a CU, so one computes while the other waits at
// its step barrier (measured: 3 stages at one workgroup per CU ran fc1 / fc2 at
// 1215 / 549 us, 2 stages at two per CU at 832 / 466 us).
#ifndef K3G_STAGES
#define K3G_STAGES 2
#endif
#ifndef K3G_WAVES_PER_EU
#define K3G_WAVES_PER_EU 2
#endif
#define K3G_STAGE_BYTES 32768
#define K3G_SAT_OFF (K3G_STAGES * K3G_STAGE_BYTES)
static_assert(K3G_STAGES == 2, "the main loop alternates two stages");

typedef __attribute__((address_space(3))) void k3g_lds_t;
typedef const __attribute__((address_space(1))) uint8_t k3g_gu8;  // global memory bytes
#define K3G_SAT_ROW(KGM) ((KGM) + 4)  // A-scale table row stride (bytes)

// The workgroup's LDS: the operand stages of the main loop, then the epilogue's
// transposition tiles (one object shared by every caller in a kernel).
#define K3G_EP_BYTES (4 * 64 * 272)  // the bf16 epilogue's four 64-row tiles
template <int KGM>
K3_DEV uint8_t* k3g_smem() {
  constexpr int kMain = K3G_SAT_OFF + 128 * K3G_SAT_ROW(KGM);
  __shared__ __attribute__((aligned(16))) uint8_t smem[kMain > K3G_EP_BYTES ? kMain : K3G_EP_BYTES];
  return smem;
}

// A rows in LDS: row r of the tile's step slice (128 bytes = 8 chunks of 16) at
// slots 8 r + (c ^ g(r)), c = chunk, g(r) = (r % 8) ^ ((r / 8) % 2).  One load
// instruction moves 8 whole 128-byte row slices (lane l of instruction q: row
// 8 q + l / 8, chunk (l % 8) ^ g(row)).  An MFMA operand read takes one chunk of
// 32 consecutive rows; LDS serves a 16-byte read in groups of 16 lanes over
// 64 four-byte banks (256 bytes), and 16 consecutive rows r0 .. r0 + 15 (r0 a
// multiple of 16) land in the 16 distinct 16-byte bank groups
// 8 (r % 2) + (c ^ g(r)) -- with g(r) = r % 8 alone, rows r and r + 8 shared a
// bank group (measured: 2-way conflicts on every A operand read).  The same
// layout is conflict-free for 8-lane groups over 32 banks (g takes 8 values on
// 8 consecutive rows).
K3_DEV int k3g_aslot(int r, int c) { return 8 * r + (c ^ ((r & 7) ^ ((r >> 3) & 1))); }

// Addresses are a wave-uniform base (scalar registers; the step moves it) plus a
// 32-bit lane offset fixed per item, so that the loads take the scalar-base form
// (global_load_lds ... v_off, s[base]) and a step costs no vector address
// arithmetic: arow[b] holds the lane's row offset plus its chunk's, lo16 = 16 l.
K3_DEV void k3g_issue_stage(uint8_t* st, const uint8_t* a, const uint32_t* arow,
                            const uint8_t* wblk, int ks, int KT, int w, uint32_t lo16) {
  const uint8_t* ak = a + (size_t)ks * K3G_KSTEP;
#pragma unroll
  for (int b = 0; b < 4; ++b)  // rows 32 w + 8 b .. + 8 of the tile (q = 4 w + b)
    __builtin_amdgcn_global_load_lds(ak + arow[b], (k3g_lds_t*)(st + (4 * w + b) * 1024), 16, 0, 0);
#pragma unroll
  for (int b = 0; b < 4; ++b) {  // B blocks: tiles 2 w, 2 w + 1, both substeps
    const int T = 2 * w + (b >> 1), s = b & 1;
    // the block's address held in scalar registers and the lane's offset added
    // last, so that the load takes the scalar-base form (left to itself the
    // compiler adds the lane offset first and the block offset to a 64-bit vector
    // address per load); then through a global-address-space pointer, which the
    // asm statement would otherwise hide
    const uint8_t* wb = wblk + ((size_t)T * KT + 2 * ks + s) * 1024;
    asm volatile("" : "+s"(wb));
    __builtin_amdgcn_global_load_lds((const k3g_gu8*)wb + lo16,
                                     (k3g_lds_t*)(st + 16384 + (T * 2 + s) * 1024), 16, 0, 0);
  }
}

template <int KGM, bool SW>
K3_DEV void k3g_lds_loop(k3_v16f (&acc)[2][4], const uint8_t* __restrict__ a,
                         const uint8_t* __restrict__ a_sf, const int* __restrict__ a_rows,
                         const uint8_t* __restrict__ wt, const uint16_t* __restrict__ wsf, int tile,
                         int cb, int e, int N, int K, int w, int lane, int wm, int wn) {
  uint8_t* lds = k3g_smem<KGM>();
  const int h = lane >> 5, j = lane & 31;
  const int KG = K / 32, KT = K / 64, KS = K / K3G_KSTEP, NT = N / 32;
  // this wave's loads: A rows 32 w + 8 b + lane / 8 (b < 4), scale rows 32 w + j
  // (byte offsets from a: every activation row offset fits in 32 bits, rows * K < 2^32)
  uint32_t arow[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int r = tile * K3G_TILE_M + 32 * w + 8 * b + (lane >> 3);
    int src = a_rows ? a_rows[r] : r;
    src = src < 0 ? 0 : src;
    // the row's offset plus that of the 16-byte chunk this lane moves
    arow[b] = (uint32_t)src * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (lane >> 3) ^ (b & 1));
  }
  uint32_t lo16 = 16u * (uint32_t)lane;
  const size_t T0 = (size_t)e * NT + cb * (K3G_TILE_N / 32);
  const uint8_t* wblk = wt + T0 * KT * 1024;
  // this wave's B scale pairs: group G = T0 / 4 + wn of its 4 tiles, 8 bytes per lane
  // per step (a wave-uniform base in scalar registers plus the lane's 8 l)
  const uint8_t* sbu = (const uint8_t*)wsf +
                       ((size_t)e * (NT / 4) + cb * (K3G_TILE_N / 128) + wn) * KS * 512;
  asm volatile("" : "+s"(sbu));  // wave-uniform: scalar registers
  uint32_t lo8 = 8u * (uint32_t)lane;
  // through a global-address-space pointer: after the asm statement the compiler
  // no longer knows where sbu points and would emit a flat load, which counts on
  // lgkmcnt as well as vmcnt, so that every wait for an LDS operand read would
  // also wait for this load (measured: 7% of fc1)
  auto sb_step = [&](int k) -> uint2 {
    return *(const uint2*)((k3g_gu8*)sbu + (size_t)k * 512 + lo8);
  };

  // the tile's A scales for all of K (KG <= KGM bytes per row), once
  // (two threads per row, each one row lookup and then independent dword loads)
  uint8_t* sat = lds + K3G_SAT_OFF;
  {
    const int row = threadIdx.x >> 1, KGd = KG / 4, half = (KGd + 1) >> 1;
    const int d0 = (threadIdx.x & 1) ? half : 0, d1 = (threadIdx.x & 1) ? KGd : half;
    const int r = tile * K3G_TILE_M + row;
    int src = a_rows ? a_rows[r] : r;
    src = src < 0 ? 0 : src;
    const uint32_t* sr = (const uint32_t*)(a_sf + (size_t)src * KG);
    uint32_t* dr = (uint32_t*)(sat + row * K3G_SAT_ROW(KGM));
#pragma unroll 8
    for (int d = d0; d < d1; ++d) dr[d] = sr[d];
  }
  uint2 sbc = sb_step(0);                               // B scale pairs of the current step
  uint2 sbq = KS > 1 ? sb_step(1) : make_uint2(0, 0);  // and of the next one
  __syncthreads();  // no stage load is in flight yet
  k3g_issue_stage(lds, a, arow, wblk, 0, KT, w, lo16);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();  // stage 0 landed for every wave
  if (KS > 1) k3g_issue_stage(lds + K3G_STAGE_BYTES, a, arow, wblk, 1, KT, w, lo16);

  // Operand reads.  The A operand of substep s: row r = 32 (2 wm + mt) + j, chunks
  // 4 s + h and 4 s + 2 + h of its 128-byte slice; the B operand: 1 KB block
  // (T, s) in lane order.
  auto rd_a = [&](const uint8_t* st, int s, int mt) -> k3_v8i {
    const int r = 32 * (2 * wm + mt) + j;
    const k3_u4 lo = *(const k3_u4*)(st + 16 * k3g_aslot(r, 4 * s + h));
    const k3_u4 hi = *(const k3_u4*)(st + 16 * k3g_aslot(r, 4 * s + 2 + h));
    return (k3_v8i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                    (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  auto rd_b = [&](const uint8_t* st, int s, int nt) -> k3_u4 {
    return *(const k3_u4*)(st + 16384 + ((4 * wn + nt) * 2 + s) * 1024 + 16 * lane);
  };
  // A scales of the step: the lane's half-wave byte shifted to bytes 0 and 2, so
  // that the MFMA's scale byte select is a per-instruction constant
  auto rd_sa = [&](int ks, int mt) -> uint32_t {
    return *(const uint32_t*)(sat + (32 * (2 * wm + mt) + j) * K3G_SAT_ROW(KGM) + 4 * ks) >>
           (8 * h);
  };
  // Both m tiles of n tile NT, substep S.  Scale bytes by the instruction's byte
  // selects: B block 4 k + 2 S + h of column j is byte 2 (NT % 2) + S of the tile
  // group's word (x: tiles 0, 1; y: tiles 2, 3), A block 4 k + 2 S + h of row j
  // byte 2 S of the shifted dword.
  auto mfma2 = [&](auto nt_c, auto s_c, const k3_v8i (&av)[2], const k3_u4& bv,
                   const uint32_t (&sa2)[2], uint2 sbw) {
    constexpr int nt = decltype(nt_c)::value, s = decltype(s_c)::value;
    constexpr int bsel = 2 * (nt & 1) + s, asel = 2 * s;
    const k3_v8i b = {(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3], 0, 0, 0, 0};
    const int sb = (int)(nt & 2 ? sbw.y : sbw.x);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      if constexpr (SW)  // weights as src0: lane (j, h) accumulates row j, 16 columns
        acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            b, av[mt], acc[mt][nt], 4, 0, bsel, sb, asel, (int)sa2[mt]);
      else
        acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            av[mt], b, acc[mt][nt], 0, 4, asel, (int)sa2[mt], bsel, sb);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // f(nt) for nt = 0..3 as compile-time constants
  auto for_nt = [&](auto&& f) {
    f(I0{});
    f(I1{});
    f(I2{});
    f(I3{});
  };

  // Software pipeline: the operands of the next substep are read from LDS behind
  // the current substep's MFMAs (A double-buffered, each B operand re-read as soon
  // as its two MFMAs are issued).  The barrier sits in the middle of the step:
  // there every wave's loads of the next stage have landed and every wave's reads
  // of the current stage are done, so the stage is refilled with step ks + 2.
  // The step body is instantiated branch-free for the steady state (MORE: a next
  // step exists; ISSUE: step ks + 2 exists) and peeled for the last two steps.
  k3_v8i a0[2], a1[2];
  k3_u4 bv[4];
  uint32_t sa[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) a0[mt] = rd_a(lds, 0, mt);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) bv[nt] = rd_b(lds, 0, nt);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) sa[mt] = rd_sa(0, mt);

  auto step = [&](int ks, auto more_c, auto issue_c) {
    constexpr bool MORE = decltype(more_c)::value, ISSUE = decltype(issue_c)::value;
    // the load offsets pass through an empty asm statement at every step, which
    // keeps the compiler from hoisting 64-bit widened copies of them out of the
    // loop (a widened copy costs a 64-bit add per load and step)
    asm volatile("" : "+v"(arow[0]), "+v"(arow[1]), "+v"(arow[2]), "+v"(arow[3]), "+v"(lo16),
                 "+v"(lo8));
    uint8_t* st = lds + (ks & 1) * K3G_STAGE_BYTES;
    const uint8_t* sn = lds + ((ks + 1) & 1) * K3G_STAGE_BYTES;
    uint32_t san[2];
    const uint2 sbw = sbc;
    // substep 0: A of substep 1 requested first, each B operand re-read behind its pair
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) a1[mt] = rd_a(st, 1, mt);
    for_nt([&](auto nt_c) {
      constexpr int nt = decltype(nt_c)::value;
      mfma2(nt_c, I0{}, a0, bv[nt], sa, sbw);
      bv[nt] = rd_b(st, 1, nt);
    });
    __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 4, 0);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      __builtin_amdgcn_sched_group_barrier(K3G_SG_MFMA, 2, 0);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 1, 0);
    }
    if constexpr (MORE) {
      // substep 0's MFMAs stay ahead of the wait (without this the compiler sinks
      // six of the eight past the barrier, which halves the loads' lead)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) asm volatile("" : "+v"(acc[mt][nt]));
      __builtin_amdgcn_s_waitcnt(0);  // this wave: stage ks + 1 landed, its reads of stage ks done
      __builtin_amdgcn_s_barrier();   // every wave
      // the copy of the landed scale pair stays behind the wait (hoisted above it,
      // it takes a wait of its own for every load in flight, the stage's included)
      asm volatile("" : "+v"(sbq));
      sbc = sbq;
      if constexpr (ISSUE) sbq = sb_step(ks + 2);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) a0[mt] = rd_a(sn, 0, mt);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) san[mt] = rd_sa(ks + 1, mt);
    }
    // substep 1; the next step's operands are read behind it, and stage ks is
    // refilled with step ks + 2 behind its first MFMA pair
    for_nt([&](auto nt_c) {
      constexpr int nt = decltype(nt_c)::value;
      mfma2(nt_c, I1{}, a1, bv[nt], sa, sbw);
      if constexpr (MORE) bv[nt] = rd_b(sn, 0, nt);
      if constexpr (ISSUE && nt == 0) {
        // the first pair goes ahead of the loads, and the loads ahead of the rest
        // (left to itself the scheduler issues them after the third pair, a
        // shorter lead for the loads)
        asm volatile("" : "+v"(acc[0][0]), "+v"(acc[1][0]));
        k3g_issue_stage(st, a, arow, wblk, ks + 2, KT, w, lo16);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int n = 1; n < 4; ++n) asm volatile("" : "+v"(acc[mt][n]));
      }
    });
    if constexpr (MORE) {
      sa[0] = san[0];
      sa[1] = san[1];
      __builtin_amdgcn_sched_group_barrier(K3G_SG_VMEM_READ, 1, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 6, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_MFMA, 2, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 1, 1);
      if constexpr (ISSUE) __builtin_amdgcn_sched_group_barrier(K3G_SG_VMEM, 8, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_MFMA, 2, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 1, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_MFMA, 2, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 1, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_MFMA, 2, 1);
      __builtin_amdgcn_sched_group_barrier(K3G_SG_DS_READ, 1, 1);
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  int ks = 0;
  for (; ks + 2 < KS; ++ks) step(ks, T_{}, T_{});
  if (ks + 1 < KS) step(ks++, T_{}, F_{});
  step(ks, F_{}, F_{});
}

// Work item of this workgroup.  The grid is (column blocks, max route tiles);
// only the live tiles' items (tile < *num_tiles) are work.  Workgroups are
// dispatched round-robin over the 8 XCDs by linear id, so items are handed out
// per XCD: the XCDs form a K3G_XT x K3G_XC grid over (live tiles, column
// blocks), XCD x taking tile part x / K3G_XC and column part x % K3G_XC in
// tile-major order.  A route tile's A rows are then fetched by K3G_XC XCDs
// and an expert's weights by about K3G_XT (each L2 keeps the operands its
// concurrent workgroups share).  Returns false for a workgroup with no item.
#ifndef K3G_XC
#define K3G_XC 2  // measured best of 1, 2, 4, 8 for fc1 and fc2
#endif
#define K3G_XT (K3G_XCDS / K3G_XC)
K3_DEV bool k3g_item(const int* __restrict__ num_tiles, int max_tiles, int& tile, int& cb) {
  const int nc = gridDim.x;
  int live = *num_tiles;
  live = live < max_tiles ? live : max_tiles;
  const int i = blockIdx.y * nc + blockIdx.x;
  const int x = i % K3G_XCDS, slot = i / K3G_XCDS;
  const int xt = x / K3G_XC, xc = x % K3G_XC;
  // this XCD's tile range [t0, t0 + nt) and column range [c0, c0 + ncx)
  const int tq = live / K3G_XT, tr = live % K3G_XT;
  const int nt = tq + (xt < tr ? 1 : 0), t0 = xt * tq + (xt < tr ? xt : tr);
  const int cq = nc / K3G_XC, cr = nc % K3G_XC;
  const int ncx = cq + (xc < cr ? 1 : 0), c0 = xc * cq + (xc < cr ? xc : cr);
  if (slot >= nt * ncx) return false;
  const int ti = slot / ncx;
  tile = t0 + ti;
  cb = c0 + (slot - ti * ncx);
  return true;
}

// Accumulates the wave's 64 x 128 block of work item (tile, cb); returns false
// when the tile's expert is out of range (the whole workgroup skips the item).
template <int KGM, bool SW>
K3_DEV bool k3g_block(k3_v16f (&acc)[2][4], const uint8_t* __restrict__ a,
                      const uint8_t* __restrict__ a_sf, const int* __restrict__ a_rows,
                      const uint8_t* __restrict__ wt, const uint16_t* __restrict__ wsf,
                      const int* __restrict__ cta_batch, int E, int N, int K, int tile, int cb,
                      int& e, int& lane, int& wm, int& wn) {
  e = cta_batch[tile];
  if (e < 0 || e >= E) return false;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  lane = threadIdx.x & 63;
  wm = w >> 1;
  wn = w & 1;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[mt][nt][q] = 0.0f;
  k3g_lds_loop<KGM, SW>(acc, a, a_sf, a_rows, wt, wsf, tile, cb, e, N, K, w, lane, wm, wn);
  return true;
}

// Runs the workgroup's item (if any): accumulates it and hands it to the
// epilogue epi(acc, tile, cb, e, lane, wm, wn).  SW: the MFMA operand roles
// swapped (the weight tile as src0, the activation rows as src1; the same
// products bit for bit), so accumulator q of lane (j, h) of tile (mt, nt) holds
// row 32 (2 wm + mt) + j, column 32 (4 wn + nt) + 8 (q / 4) + 4 h + q % 4.
template <int KGM, bool SW = false, class Epi>
K3_DEV void k3g_items(const uint8_t* __restrict__ a, const uint8_t* __restrict__ a_sf,
                      const int* __restrict__ a_rows, const uint8_t* __restrict__ wt,
                      const uint16_t* __restrict__ wsf, const int* __restrict__ num_tiles,
                      const int* __restrict__ cta_batch, int E, int N, int K, int max_tiles,
                      Epi&& epi) {
  int tile, cb, e, lane, wm, wn;
  if (!k3g_item(num_tiles, max_tiles, tile, cb)) return;
  k3_v16f acc[2][4];
  if (!k3g_block<KGM, SW>(acc, a, a_sf, a_rows, wt, wsf, cta_batch, E, N, K, tile, cb, e, lane, wm,
                          wn))
    return;
  epi(acc, tile, cb, e, lane, wm, wn);
}

// Row of accumulator register q of m tile mt, within the route tile.
K3_DEV int k3g_out_row(int wm, int mt, int q, int h) {
  return 64 * wm + 32 * mt + 8 * (q >> 2) + 4 * h + (q & 3);
}

#define K3G_PARAMS                                                                          \
  const uint8_t *__restrict__ a, const uint8_t *__restrict__ a_sf,                          \
      const int *__restrict__ a_rows, const uint8_t *__restrict__ wt,                       \
      const uint16_t *__restrict__ wsf, const int *__restrict__ num_tiles,                  \
      const int *__restrict__ cta_batch, int E, int N, int K, int max_tiles

template <int KGM>
K3_DEV void k3g_gemm_f32(K3G_PARAMS, float* __restrict__ out) {
  k3g_items<KGM>(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
                 [&](k3_v16f(&acc)[2][4], int tile, int cb, int e, int lane, int wm, int wn) {
    const int h = lane >> 5, j = lane & 31;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int col = cb * K3G_TILE_N + 128 * wn + 32 * nt + j;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const size_t row = (size_t)tile * K3G_TILE_M + k3g_out_row(wm, mt, q, h);
          out[row * N + col] = acc[mt][nt][q];
        }
      }
  });
}

// Epilogue transposition: each wave writes its 64 x 128 block (bf16) to its own
// LDS tile, row stride K3G_EP_ROW bytes (padded so that the column writes of the
// two half-waves and the 16-byte row reads hit different banks); lane l then
// owns row l and stores it with 16-byte writes.
#define K3G_EP_ROW 272
#define K3G_EP_TILE (64 * K3G_EP_ROW)

template <int KGM>
K3_DEV void k3g_gemm_bf16(K3G_PARAMS, uint16_t* __restrict__ out) {
  k3g_items<KGM>(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
                 [&](k3_v16f(&acc)[2][4], int tile, int cb, int e, int lane, int wm, int wn) {
    const int h = lane >> 5, j = lane & 31;
    __syncthreads();  // every wave is done with the operand stages
    uint8_t* wl = k3g_smem<KGM>() + (threadIdx.x >> 6) * K3G_EP_TILE;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int r = 32 * mt + 8 * (q >> 2) + 4 * h + (q & 3);
          *(uint16_t*)(wl + r * K3G_EP_ROW + 2 * (32 * nt + j)) =
              (uint16_t)k3_pack_bf2(acc[mt][nt][q], 0.0f);
        }
    __syncthreads();
    uint16_t* orow = out + ((size_t)tile * K3G_TILE_M + 64 * wm + lane) * N + cb * K3G_TILE_N +
                     128 * wn;
#pragma unroll
    for (int c = 0; c < 16; ++c)
      k3_st16(orow + 8 * c, *(const k3_u4*)(wl + lane * K3G_EP_ROW + 16 * c));
  });
}

// fc1 epilogue, on the swapped accumulator layout (no LDS): lane (j, h) holds,
// for each m tile and activation tile (logical tiles 2 p: up, and 2 p + 1: gate,
// within the wave's four), the 16 activation columns 8 (q / 4) + 4 h + q % 4 of
// one row.  The 32-column MX block of (row, p) is the lane pair (l, l ^ 32):
// the block amax takes one exchange (v_permlane32_swap), the e4m3 codes are
// quantised in registers as kern_k3_moe_quant does (block amax of the bf16
// activations, E8M0 exponent, e4m3 of x * 2^-e), and two exchanges of code
// dwords leave lane (j, h) with columns 16 h .. + 16 of the block: one 16-byte
// store per lane and block.  Returns the block's E8M0 byte.  FORM 0: the K3
// constants (alpha 4, beta 25), k3_situ; 1: alpha 4, general beta; 2: general
// alpha and beta.  A template parameter, so that the choice is one branch per
// item rather than one per activation (which would cut the unrolled block into
// a basic block per activation).
template <int FORM>
K3_DEV uint32_t k3g_situ_block(const k3_v16f& up, const k3_v16f& gate, float al, float ial,
                               float be, float ibe, uint8_t* __restrict__ o, int h) {
  // bf16 activations in q order, as f32; their block amax in f32 (the max of
  // bf16 values is a bf16 value, NaN ignored as in kern_k3_moe_quant)
  float xr[16];
  float am = 0.0f;
  auto act = [&](auto expf_c) {
    constexpr bool EXPF = decltype(expf_c)::value;
#pragma unroll
    for (int q = 0; q < 16; q += 2) {
      const uint32_t u2 = k3_pack_bf2(up[q], up[q + 1]);
      const uint32_t g2 = k3_pack_bf2(gate[q], gate[q + 1]);
      float x[2];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const float u = d ? k3_bf_hi(u2) : k3_bf_lo(u2);
        const float g = d ? k3_bf_hi(g2) : k3_bf_lo(g2);
        if constexpr (FORM == 0) x[d] = k3_situ_fused<EXPF>(g, u);
        else if constexpr (FORM == 1) x[d] = k3_situ_gate(g) * k3_situ_up_b<EXPF>(u, be, ibe);
        else x[d] = k3_situ_gate_a(g, al, ial) * k3_situ_up_b<EXPF>(u, be, ibe);
      }
      const uint32_t xb = k3_pack_bf2(x[0], x[1]);
      xr[q] = k3_bf_lo(xb);
      xr[q + 1] = k3_bf_hi(xb);
      am = __builtin_fmaxf(am, __builtin_fabsf(xr[q]));
      am = __builtin_fmaxf(am, __builtin_fabsf(xr[q + 1]));
    }
  };
  // the up factor's exponential form only when some lane of the wave has an up
  // value past the series range (the bf16 landing is monotone, so the lane's
  // largest landed |u| is the landing of its largest |u|)
  float um = 0.0f;
#pragma unroll
  for (int q = 0; q < 16; ++q) um = __builtin_fmaxf(um, __builtin_fabsf(up[q]));
  um = k3_bf_lo(k3_pack_bf2(um, 0.0f));
  const bool ser = FORM == 0 ? k3_situ_up_series_ok(um) : k3_situ_up_b_series_ok(um, ibe);
  if (ser) act(std::false_type{});
  else act(std::true_type{});
  uint32_t mx = __float_as_uint(am) >> 16, my = mx;
  k3g_swap(mx, my);  // mx: lane l % 32's amax, my: lane 32 + l % 32's
  const int ex = k3_e8m0_exp(mx > my ? mx : my);
  const float(&x0)[8] = *reinterpret_cast<const float(*)[8]>(&xr[0]);
  const float(&x1)[8] = *reinterpret_cast<const float(*)[8]>(&xr[8]);
  const k3_u2 c0 = k3_f8_to_e4m3(x0, ex), c1 = k3_f8_to_e4m3(x1, ex);
  // code dwords: columns 4 h + 0..3, 8 + 4 h.., 16 + 4 h.., 24 + 4 h..
  uint32_t d0 = c0[0], d1 = c0[1], d2 = c1[0], d3 = c1[1];
  k3g_swap(d0, d2);
  k3g_swap(d1, d3);
  k3_st16(o + 16 * h, (k3_u4){d0, d2, d1, d3});
  return (uint32_t)(ex + 127);
}

template <int KGM>
K3_DEV void k3g_gemm_situ_mx(K3G_PARAMS, uint8_t* __restrict__ out_q, uint8_t* __restrict__ out_sf,
                             const float* __restrict__ alpha, const float* __restrict__ beta) {
  k3g_items<KGM, true>(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
                       [&](k3_v16f(&acc)[2][4], int tile, int cb, int e, int lane, int wm, int wn) {
    const int h = lane >> 5, j = lane & 31;
    const float al = alpha[e], be = beta[e];
    const float ial = 1.0f / al, ibe = 1.0f / be;
    // the K3 constants (every layer's alpha = 4, beta = 25) take k3_situ, which
    // computes the same values as the general form with fewer instructions
    const int form = al == 4.0f ? (be == 25.0f ? 0 : 1) : 2;
    const int NA = N / 2;                 // activation columns
    const int col0 = 64 * (2 * cb + wn);  // this wave's first activation column
    auto blocks = [&](auto form_c) {
      constexpr int FORM = decltype(form_c)::value;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const size_t row = (size_t)tile * K3G_TILE_M + 64 * wm + 32 * mt + j;
        uint32_t sfp = 0;
#pragma unroll
        for (int p = 0; p < 2; ++p)
          sfp |= k3g_situ_block<FORM>(acc[mt][2 * p], acc[mt][2 * p + 1], al, ial, be, ibe,
                                     out_q + row * NA + col0 + 32 * p, h)
                 << (8 * p);
        if (h == 0) *(uint16_t*)(out_sf + row * (NA / 32) + col0 / 32) = (uint16_t)sfp;
      }
    };
    if (form == 0) blocks(std::integral_constant<int, 0>{});
    else if (form == 1) blocks(std::integral_constant<int, 1>{});
    else blocks(std::integral_constant<int, 2>{});
  });
}

// The fc1 entry's tiling with its accumulators stored as f32 instead of the
// SiTU-GLU + MXFP8 epilogue: the same items, item split and swapped operand roles
// as kern_k3h_moe_gemm_situ_mx, so a check of these accumulators (against the
// other f32 entries, bit for bit, and as the input of the CPU epilogue) checks
// the shipped fc1 kernel's products on every row.  Lane (j, h) of tile (mt, nt)
// holds row 32 (2 wm + mt) + j and columns 32 (4 wn + nt) + 8 g + 4 h + 0..3 in
// accumulators 4 g .. 4 g + 3.
template <int KGM>
K3_DEV void k3g_gemm_situ_acc(K3G_PARAMS, float* __restrict__ out) {
  k3g_items<KGM, true>(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
                       [&](k3_v16f(&acc)[2][4], int tile, int cb, int, int lane, int wm, int wn) {
    const int h = lane >> 5, j = lane & 31;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float* orow = out + ((size_t)tile * K3G_TILE_M + 32 * (2 * wm + mt) + j) * N;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        float* o = orow + cb * K3G_TILE_N + 32 * (4 * wn + nt) + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(k3_u4*)(o + 8 * g) = (k3_u4){__float_as_uint(acc[mt][nt][4 * g]), __float_as_uint(acc[mt][nt][4 * g + 1]),
                                         __float_as_uint(acc[mt][nt][4 * g + 2]), __float_as_uint(acc[mt][nt][4 * g + 3])};
      }
    }
  });
}

// Entries: K <= 3584 (A-scale table of 112 bytes per row, two workgroups per CU)
// and, suffix _w, K <= 7168 (224 bytes per row, one workgroup per CU).
#define K3G_ARGS a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles
#define K3G_ENTRIES(SUF, KGM)                                                                    \
  extern "C" __global__ void __launch_bounds__(256, K3G_WAVES_PER_EU)                            \
      kern_k3h_moe_gemm_f32##SUF(K3G_PARAMS, float* __restrict__ out) {                          \
    k3g_gemm_f32<KGM>(K3G_ARGS, out);                                                            \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(256, K3G_WAVES_PER_EU)                            \
      kern_k3h_moe_gemm_bf16##SUF(K3G_PARAMS, uint16_t* __restrict__ out) {                      \
    k3g_gemm_bf16<KGM>(K3G_ARGS, out);                                                           \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(256, K3G_WAVES_PER_EU)                            \
      kern_k3h_moe_gemm_situ_mx##SUF(K3G_PARAMS, uint8_t* __restrict__ out_q,                    \
                                     uint8_t* __restrict__ out_sf,                               \
                                     const float* __restrict__ alpha,                            \
                                     const float* __restrict__ beta) {                           \
    k3g_gemm_situ_mx<KGM>(K3G_ARGS, out_q, out_sf, alpha, beta);                                 \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(256, K3G_WAVES_PER_EU)                            \
      kern_k3h_moe_gemm_situ_acc##SUF(K3G_PARAMS, float* __restrict__ out) {                     \
    k3g_gemm_situ_acc<KGM>(K3G_ARGS, out);                                                       \
  }
K3G_ENTRIES(, 112)
K3G_ENTRIES(_w, 224)

#include "k3_gemm_wide.h"
K3W_ENTRIES
