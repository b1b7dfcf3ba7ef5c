// Wide items for the MoE expert GEMMs (module k3h_moe_gemm, included by
// k3h_moe_gemm.hip after the 256-column kernels, whose layouts and helpers it
// shares).  Entries kern_k3h_moe_gemm2_f32 and kern_k3h_moe_gemm2_bf16 compute
// the same products as kern_k3h_moe_gemm_f32 / _bf16 (bit for bit: the same
// MFMA sequence per output element), for N % 512 == 0 and 256 <= K <= 3584; the
// fc1 form (SiTU-GLU + MXFP8 epilogue) stays on the 4-wave kernels, whose second
// workgroup per CU runs its MFMAs while the first evaluates the activation.
//
// Work item: route tile t (128 rows) x one 512-column block.  Persistent: one
// 512-thread workgroup (8 waves, two per SIMD) per CU, grid a multiple of 8;
// workgroup i serves XCD i % 8 (workgroups are dispatched round-robin over the
// XCDs) and takes every (grid / 8)-th item of that XCD's part of the items (the
// XCDs split the tile-major item list into eight equal contiguous ranges),
// skipping tiles whose expert is out of range.  Per K step of 128 the
// workgroup brings 48 KB of operands into LDS (16 KB of A rows, 32 KB of B
// tiles), 25% fewer bytes per FLOP than the 128 x 256 items of the 4-wave
// kernels, whose operand traffic through the CU's vector-memory path bounds
// them.  The step pipeline runs on across items: the loads of an item's first
// two steps go out during the previous item's last two, so an item starts
// without a load wait and the grid is launched once.
//
// Operand roles are swapped relative to the 4-wave kernels: the matrix-core
// src0 operand is the e2m1 weight tile (32 output columns n x 64 k), src1 the
// e4m3 activation rows (32 rows x 64 k), so accumulator VGPR q of lane
// l = (j = l % 32, h = l / 32) of MFMA tile (mt, nt) holds
//   C[row 32 mt + j][n 32 nt + 8 (q / 4) + 4 h + q % 4]
// (both operands keep their lane layouts: lane (i, h) supplies row / column i
// over the 32-blocks h, as measured for the 4-wave kernels).  A lane then holds
// 16 columns of one row, and after one exchange of 8 dwords with lane l ^ 32
// (v_permlane32_swap) 16 consecutive columns: the epilogues need no LDS.
//
// Waves: w = 4 g + wq (g = wave group, wq < 4) owns rows 64 g .. + 64 and
// columns 128 wq .. + 128 of the item (2 x 4 MFMA tiles, 128 accumulators).
// Group g's waves sit one per SIMD (measured: waves w and w + 4 share a SIMD).
// Schedule ("ping-pong"): each step is a memory phase M (issue the
// direct-to-LDS loads of the step two ahead; LDS -> registers: this step's A /
// B operands and scales) and a compute phase C (the step's 16 MFMAs).  The
// groups run one phase apart, every phase ending at a workgroup barrier, so on
// every SIMD one wave computes while the other moves operands:
//   phase 2s: group 0 M(s), group 1 C(s - 1);  phase 2s + 1: group 0 C(s),
//   group 1 M(s)   (s counts the workgroup's steps over all its items).
// An item's epilogue runs at the head of the group's next memory phase.
// Three stages: the item's stage i % 3 (physical stage (rot + i) % 3, rot
// advancing by K / 128 per item) holds its step i; the loads of step s + 2 go
// to the stage of step s - 1, last read in phases 2s - 2 and 2s - 1, and must
// have landed before phase 2s + 4: every wave waits for its loads of step s + 1
// before the barrier that ends phase 2s + 1 (group 0 after C(s), group 1 after
// M(s)), leaving only those issued in M(s) in flight.  Every load of the step
// loop is a direct-to-LDS load, so the compiler adds no waits of its own.
// Stage bytes:
//   A   16 KB: 128 rows' 128-byte slices, swizzled as k3g_aslot;
//   B   32 KB: 16 tiles x 2 substeps, 1 KB each in MFMA lane order;
//   SA  512 B: the 128 rows' E8M0 bytes of the step (4 blocks per row, a dword);
//   SB  2 KB:  the 4 tile groups' B-scale pairs of the step (64 lanes x 8 B each).
// LDS: 3 x 51,712 = 155,136 bytes.
#pragma once

typedef float k3w_f4 __attribute__((ext_vector_type(4)));

#define K3W_TILE_N 512
#define K3W_A_BYTES 16384
#define K3W_SA_OFF 49152
#define K3W_SB_OFF (K3W_SA_OFF + 512)
#define K3W_STAGE_BYTES (K3W_SB_OFF + 2048)
#define K3W_LDS_BYTES (3 * K3W_STAGE_BYTES)
static_assert(K3W_LDS_BYTES <= 163840, "one workgroup's LDS");

K3_DEV uint8_t* k3w_smem() {
  __shared__ __attribute__((aligned(16))) uint8_t smem[K3W_LDS_BYTES];
  return smem;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8); unnamed counters at their maximum.
#define K3W_VMCNT(n) (((n) & 15) | (((n) >> 4) << 14) | 0x0f70)
#define K3W_LGKMCNT0 0xc07f

// Waits until at most n of this wave's vector-memory operations are in flight
// (n: the operations of the latest memory phase, 0 or 8).
K3_DEV void k3w_wait_vm(int n) {
  if (n == 8) __builtin_amdgcn_s_waitcnt(K3W_VMCNT(8));
  else __builtin_amdgcn_s_waitcnt(K3W_VMCNT(0));
}

// One work item (wave-uniform): its slot in the workgroup's list, route tile,
// 512-column block and expert.
struct K3wItem {
  int slot, tile, cb, e;
};

// This workgroup's share of the items: slots c, c + ncu, ... below nslots of
// its XCD's item range [i0, i0 + nslots).  Items are numbered tile-major over
// the live tiles (item = tile * nc + column block) and the eight XCDs take
// equal contiguous ranges of them, so no CU has more than ceil(items / 8 / ncu)
// items whatever the live tile count (a split by whole tiles adds a round
// whenever the remainder tiles' column blocks overflow it: 290 live tiles, 7
// column blocks, 32 CUs per XCD gave 9 items to some CUs instead of 8); a tile
// at a range boundary has its column blocks on two XCDs.
struct K3wList {
  int i0, nc, nslots, c, ncu, E;
  const int* cta_batch;
  // the first item at slot >= s (s = c + k ncu) whose expert is in range;
  // slot >= nslots: none
  K3_DEV K3wItem at(int s) const {
    for (; s < nslots; s += ncu) {
      const int item = i0 + s;
      const int tile = item / nc, e = cta_batch[tile];
      if (e >= 0 && e < E) return {s, tile, item - tile * nc, e};
    }
    return {nslots, 0, 0, 0};
  }
  K3_DEV bool live(const K3wItem& it) const { return it.slot < nslots; }
};

K3_DEV K3wList k3w_list(const int* __restrict__ num_tiles, const int* __restrict__ cta_batch,
                        int max_tiles, int nc, int E) {
  int live = *num_tiles;
  live = live < max_tiles ? live : max_tiles;
  const int x = blockIdx.x % K3G_XCDS, ncu = gridDim.x / K3G_XCDS;
  const long long total = (long long)live * nc;
  const int i0 = (int)(total * x / K3G_XCDS), i1 = (int)(total * (x + 1) / K3G_XCDS);
  return {i0, nc, i1 - i0, (int)blockIdx.x / K3G_XCDS, ncu, E, cta_batch};
}

struct K3wOps {
  k3_v8i av[2][2];  // [mt][substep]
  k3_u4 bv[4][2];   // [nt][substep]
  uint32_t sa[2];   // A-scale dword (blocks 4 k .. 4 k + 3) of m tile mt's row
  uint2 sb;         // the 4 tiles' B-scale pairs (tile u: bits 16 (u % 2) of x / y)
};

// Runs the workgroup's items; epi(acc, tile, cb, e) takes each item's
// accumulators.  One entry serves every K: the step loop runs KS = K / 128 steps
// per item with the stage index S held at run time (S advances modulo 3 each
// step), and the item's stage s lives in physical stage (rot + s) % 3, rot
// advancing by KS per item, so the next item's first two steps load into the
// stages the current item's last two steps free.
template <class Epi>
K3_DEV void k3w_run(const uint8_t* __restrict__ a, const uint8_t* __restrict__ a_sf,
                    const int* __restrict__ a_rows, const uint8_t* __restrict__ wt,
                    const uint16_t* __restrict__ wsf, const int* __restrict__ num_tiles,
                    const int* __restrict__ cta_batch, int E, int N, int K, int max_tiles,
                    Epi&& epi) {
  const K3wList L = k3w_list(num_tiles, cta_batch, max_tiles, N / K3W_TILE_N, E);
  K3wItem it = L.at(L.c);
  if (!L.live(it)) return;  // no work for this workgroup (uniform)
  K3wItem nx = L.at(it.slot + L.ncu);

  uint8_t* lds = k3w_smem();
  // wave-uniform indices in scalar registers (the group branches below are scalar)
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, h = lane >> 5, j = lane & 31;
  const int g = w >> 2, wq = w & 3;
  const int KG = K / 32, KT = K / 64, KS = K / K3G_KSTEP, NT = N / 32;
  const uint8_t* wsf8 = (const uint8_t*)wsf;

  // This lane's source rows of item t: the A-row byte offsets of its two row-slice
  // loads (rows 8 q + l / 8, q = 2 w, 2 w + 1, plus the lane's chunk) and the
  // A-scale byte offset of row 16 w + l % 16 (every activation row offset fits in
  // 32 bits: rows * K < 2^32).
  auto rows_of = [&](const K3wItem& t, uint32_t (&ar)[2], uint32_t& sr) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int q = 2 * w + b;
      const int r = t.tile * K3G_TILE_M + 8 * q + (lane >> 3);
      int src = a_rows ? a_rows[r] : r;
      src = src < 0 ? 0 : src;
      // the row's offset plus that of the 16-byte chunk this lane moves
      ar[b] = (uint32_t)src * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (lane >> 3) ^ (q & 1));
    }
    const int r = t.tile * K3G_TILE_M + 16 * w + (lane & 15);
    int src = a_rows ? a_rows[r] : r;
    src = src < 0 ? 0 : src;
    sr = (uint32_t)src * (uint32_t)KG;
  };
  // This wave's 8 direct-to-LDS loads of step k of item t into stage st: A row
  // slices q = 2 w, 2 w + 1 (lane l: row 8 q + l / 8, the chunk that lands at slot
  // 8 r + l % 8); B blocks 4 w .. 4 w + 3 (tile b / 2, substep b % 2); lanes 0-15:
  // the A scales of rows 16 w + l and 16 bytes of B-scale group w / 2.
  // Every address is a wave-uniform base (scalar registers; the step moves it)
  // plus a 32-bit lane offset fixed per item, so that the loads take the
  // scalar-base form (global_load_lds ... v_off, s[base]) and a step costs no
  // vector address arithmetic.  The offsets pass through an empty asm statement
  // at every step (step() below), which keeps the compiler from hoisting 64-bit
  // widened copies of them out of the step loop (a widened copy costs a 64-bit
  // add per load and step).
  uint32_t lo16 = 16u * (uint32_t)lane;
  auto issue = [&](uint8_t* st, const K3wItem& t, const uint32_t (&ar)[2], uint32_t sr, int k) {
    const uint8_t* ak = a + (size_t)k * K3G_KSTEP;
#pragma unroll
    for (int b = 0; b < 2; ++b)
      __builtin_amdgcn_global_load_lds(ak + ar[b], (k3g_lds_t*)(st + (2 * w + b) * 1024), 16, 0, 0);
    const uint8_t* wblk = wt + ((size_t)t.e * NT + (size_t)t.cb * (K3W_TILE_N / 32)) * KT * 1024;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int blk = 4 * w + b;
      const uint8_t* wb = wblk + ((size_t)(blk >> 1) * KT + 2 * k + (blk & 1)) * 1024;
      __builtin_amdgcn_global_load_lds(wb + lo16, (k3g_lds_t*)(st + K3W_A_BYTES + blk * 1024), 16,
                                       0, 0);
    }
    const uint8_t* sbg =
        wsf8 + (((size_t)t.e * (NT / 4) + (size_t)t.cb * (K3W_TILE_N / 128) + (w >> 1)) * KS + k) *
                   512 +
        256 * (w & 1);
    if (lane < 16) {
      __builtin_amdgcn_global_load_lds(a_sf + (size_t)4 * k + sr,
                                       (k3g_lds_t*)(st + K3W_SA_OFF + 64 * w), 4, 0, 0);
      __builtin_amdgcn_global_load_lds(sbg + lo16, (k3g_lds_t*)(st + K3W_SB_OFF + 256 * w), 16, 0,
                                       0);
    }
  };

  uint32_t arow[2], srow, arow_n[2] = {0, 0}, srow_n = 0;
  rows_of(it, arow, srow);
  int rot = 0;  // physical stage of the item's stage 0
  // physical stage of the current item's stage S
  auto stage = [&](int S) -> uint8_t* {
    const int p = rot + S;
    return lds + (p >= 3 ? p - 3 : p) * K3W_STAGE_BYTES;
  };
  // prologue: the first item's first two steps
  issue(stage(0), it, arow, srow, 0);
  issue(stage(1), it, arow, srow, 1);
  if (L.live(nx)) rows_of(nx, arow_n, srow_n);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the first two stages are in place

  k3_v16f acc[2][4];
  auto zero = [&]() {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[mt][nt][q] = 0.0f;
  };
  zero();

  K3wOps op;
  const int r0 = 64 * g + j;  // this lane's row in m tile 0 (m tile 1: + 32)
  // The lane's A slots: row r0 + 32 mt sits 256 slots (4096 bytes) after row r0
  // in the same chunk order (the swizzle depends on r % 16 only), so the four
  // chunks' byte offsets serve both m tiles.
  int aoff[2][2];  // [substep][low / high chunk]
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    aoff[s][0] = 16 * k3g_aslot(r0, 4 * s + h);
    aoff[s][1] = 16 * k3g_aslot(r0, 4 * s + 2 + h);
  }
  auto memory = [&](const uint8_t* st) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint8_t* plo = st + aoff[s][0];
      const uint8_t* phi = st + aoff[s][1];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const k3_u4 lo = *(const k3_u4*)(plo + 4096 * mt);
        const k3_u4 hi = *(const k3_u4*)(phi + 4096 * mt);
        op.av[mt][s] = (k3_v8i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                                (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        op.bv[nt][s] =
            *(const k3_u4*)(st + K3W_A_BYTES + ((4 * wq + nt) * 2 + s) * 1024 + 16 * lane);
    // A scales: the lane's half-wave byte moved to bytes 0 and 2 (one shift per m
    // tile), so that the MFMA's scale byte select is a per-instruction constant
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      op.sa[mt] = *(const uint32_t*)(st + K3W_SA_OFF + 4 * (r0 + 32 * mt)) >> (8 * h);
    op.sb = *(const uint2*)(st + K3W_SB_OFF + 512 * wq + 8 * lane);
  };
  // The accumulators pass through empty volatile asm at both edges of a compute
  // phase, so the phase's MFMAs can move neither above its opening barrier nor
  // below its closing one (IR-level code motion ignores sched_barrier).
  auto pin = [&]() {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) asm volatile("" : "+v"(acc[mt][nt]));
  };
  // One substep s of n tile NT for both m tiles.  Scale bytes are picked by the
  // instruction's byte selects: B block 4 k + 2 s + h of column j is byte
  // 2 (NT % 2) + s of the tile group's word, A block 4 k + 2 s + h of row j byte
  // 2 s of the shifted dword.
  auto mfma2 = [&](auto nt_c, auto s_c) {
    constexpr int nt = decltype(nt_c)::value, s = decltype(s_c)::value;
    const k3_u4& b = op.bv[nt][s];
    const k3_v8i bw = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};
    const uint32_t sb = nt & 2 ? op.sb.y : op.sb.x;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          bw, op.av[mt][s], acc[mt][nt], 4, 0, 2 * (nt & 1) + s, (int)sb, 2 * s, (int)op.sa[mt]);
  };
  auto compute = [&]() {
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    mfma2(I0{}, I0{}); mfma2(I1{}, I0{}); mfma2(I2{}, I0{}); mfma2(I3{}, I0{});
    mfma2(I0{}, I1{}); mfma2(I1{}, I1{}); mfma2(I2{}, I1{}); mfma2(I3{}, I1{});
  };

  bool more = L.live(nx);
  // One step: memory phase (issue the loads of the step two ahead: KIND 1 the
  // current item's step i + 2, KIND 2 the next item's step i + 2 - KS, if any;
  // then this step's operands from stage S) and compute phase.  Group 1 ends its
  // memory phase and group 0 its compute phase with this wave's loads of the next
  // step landed (those just issued left in flight).
  auto step = [&](int i, int S) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(arow[0]), "+v"(arow[1]), "+v"(srow), "+v"(lo16));
    asm volatile("" : "+v"(arow_n[0]), "+v"(arow_n[1]), "+v"(srow_n));
    int nvm = 0;
    const int S2 = S == 0 ? 2 : S - 1;  // (S + 2) % 3
    if (i + 2 < KS) {
      issue(stage(S2), it, arow, srow, i + 2);
      nvm = 8;
    } else if (more) {
      issue(stage(S2), nx, arow_n, srow_n, i + 2 - KS);
      nvm = 8;
    }
    memory(stage(S));
    __builtin_amdgcn_s_waitcnt(K3W_LGKMCNT0);
    if (g == 1) k3w_wait_vm(nvm);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pin();
    compute();
    pin();
    __builtin_amdgcn_sched_barrier(0);
    if (g == 0) k3w_wait_vm(nvm);
    if (g == 0 || i + 1 < KS || more) {  // group 1's last compute phase ends the run
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  if (g == 1) __builtin_amdgcn_s_barrier();  // group 1 runs one phase behind
  for (;;) {
    int S = 0;
    for (int i = 0; i < KS; ++i) {
      step(i, S);
      S = S == 2 ? 0 : S + 1;
    }
    // the item's epilogue (registers and stores only), then the next item
    epi(acc, it.tile, it.cb, it.e);
    if (!more) break;
    zero();
    it = nx;
    arow[0] = arow_n[0];
    arow[1] = arow_n[1];
    srow = srow_n;
    rot = (rot + KS) % 3;
    nx = L.at(it.slot + L.ncu);
    more = L.live(nx);
    if (more) rows_of(nx, arow_n, srow_n);
  }
}

// Output row of m tile mt for this lane, and the item's first column of n tile nt.
#define K3W_LANE_ROW(mt)                                                                     \
  ((size_t)tile * K3G_TILE_M + 64 * ((threadIdx.x >> 6) >> 2) + 32 * (mt) + (threadIdx.x & 31))
#define K3W_TILE_COL(nt) (cb * K3W_TILE_N + 32 * (4 * ((threadIdx.x >> 6) & 3) + (nt)))

K3_DEV void k3w_gemm_f32(K3G_PARAMS, float* __restrict__ out) {
  k3w_run(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
          [&](k3_v16f(&acc)[2][4], int tile, int cb, int) {
    const int h = (threadIdx.x >> 5) & 1;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        float* o = out + K3W_LANE_ROW(mt) * N + K3W_TILE_COL(nt) + 4 * h;
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
          *(k3w_f4*)(o + 8 * gq) = (k3w_f4){acc[mt][nt][4 * gq], acc[mt][nt][4 * gq + 1],
                                            acc[mt][nt][4 * gq + 2], acc[mt][nt][4 * gq + 3]};
      }
  });
}

// bf16 out: the lane's columns 8 gq + 4 h + c as four 2-dword groups D[gq];
// after swap(D0, D2) and swap(D1, D3) the lower half-wave holds columns 0..15
// and the upper 16..31 of the tile, in the register order below.
K3_DEV void k3w_gemm_bf16(K3G_PARAMS, uint16_t* __restrict__ out) {
  k3w_run(a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch, E, N, K, max_tiles,
          [&](k3_v16f(&acc)[2][4], int tile, int cb, int) {
    const int h = (threadIdx.x >> 5) & 1;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        uint32_t d[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) d[k] = k3_pack_bf2(acc[mt][nt][2 * k], acc[mt][nt][2 * k + 1]);
        k3g_swap(d[0], d[4]);
        k3g_swap(d[1], d[5]);
        k3g_swap(d[2], d[6]);
        k3g_swap(d[3], d[7]);
        // Lane (j, h) now holds 16-byte chunks 2 h (X) and 2 h + 1 (Y) of row j's 64
        // bytes.  Lanes j and j ^ 1 (DPP quad_perm [1,0,3,2]) trade one chunk, the
        // even lane its Y, the odd lane its X, so that each store writes 16 rows x 64
        // contiguous bytes (the even rows, then the odd ones) instead of 32 rows x
        // two 16-byte pieces: half the write requests (measured: fc2 4% faster).
        const int p = threadIdx.x & 1;
        const k3_u4 X = {d[0], d[1], d[4], d[5]}, Y = {d[2], d[3], d[6], d[7]};
        const k3_u4 snd = p ? X : Y;
        k3_u4 rcv;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          rcv[c] = (uint32_t)__builtin_amdgcn_mov_dpp((int)snd[c], K3_DPP_QP_1032, 0xf, 0xf, false);
        uint16_t* o = out + (K3W_LANE_ROW(mt) & ~(size_t)1) * N + K3W_TILE_COL(nt) + 8 * (2 * h + p);
        k3_st16(o, p ? rcv : X);      // row j & ~1: chunk 2 h + p
        k3_st16(o + N, p ? Y : rcv);  // row j | 1
      }
  });
}

#define K3W_ENTRIES                                                                              \
  extern "C" __global__ void __launch_bounds__(512, 1)                                           \
      kern_k3h_moe_gemm2_f32(K3G_PARAMS, float* __restrict__ out) {                              \
    k3w_gemm_f32(K3G_ARGS, out);                                                                 \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(512, 1)                                           \
      kern_k3h_moe_gemm2_bf16(K3G_PARAMS, uint16_t* __restrict__ out) {                          \
    k3w_gemm_bf16(K3G_ARGS, out);                                                                \
  }
