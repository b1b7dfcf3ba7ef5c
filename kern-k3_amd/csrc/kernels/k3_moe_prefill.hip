// Module k3_moe_prefill_v{3,4}+...: the MoE prefill memory-bound family on gfx950.
//
//   kern_k3_moe_quant(x, q, sf, rows, cols)       grid ceil(rows*cols/32/256), block 256
//   kern_k3_moe_route_count(ids, T, rank, E, blockcount)      grid ceil(T/256), block 256
//   kern_k3_moe_route_tables(blockcount, blocks, E, tile, blockoff, cta_batch,
//       cta_limit, num_non_exiting, total_padded, route_map)  grid 1, block 1024
//   kern_k3_moe_route_scatter(ids, blockoff, T, rank, E, route_map, exp2perm)
//                                                   grid ceil(T/256), block 32*SCATTER_WARPS
//   kern_k3_moe_finalize(fc2, exp2perm, wts, out, T, cols)     grid ceil(T/2), block 128
//   kern_k3_moe_w_shuffle(src, dst, experts, n, row_bytes, gated)
//   kern_k3_moe_sf_shuffle(src, dst, experts, n, kg, gated)
//
// Entry names, parameter order and launch geometry are the reference module's
// (k3_moe_prefill_v4.cu:27-80; manifest ops moe_quant, moe_route_count,
// moe_route_tables, moe_route_scatter, moe_finalize at k3-tp4-prefill-16k.json
// 404926, 404991, 405046, 405120, 405686).  Defines as in the module keys:
// TOPK (16), EP_RANKS (4), EP_STRIDED, TILE_SHIFT (tile = 1 << TILE_SHIFT,
// otherwise the run-time `tile`), SCATTER_WARPS (block 32 * SCATTER_WARPS).
//
// Plus one operator with no reference entry (module key k3_moe_prefill_v4+...):
//   k3h_moe_permute_mx(q, sf, route_map, total_padded, max_rows, cols, pq, psf)
//       grid min(ceil(max_rows / 4), 16384), block 256: pq[r] = q[route_map[r]],
//       psf[r] = sf[route_map[r]] for r < min(*total_padded, max_rows) (the
//       reference gathers these rows inside moe_fc1).
#include "k3_mx.h"

#ifndef TOPK
#define TOPK 16
#endif
#ifndef EP_RANKS
#define EP_RANKS 4
#endif
#ifndef SCATTER_WARPS
#define SCATTER_WARPS 8
#endif
#define MAX_E 64
#define ROUTE_BLOCK 256
#define ROUTE_IDS (ROUTE_BLOCK * TOPK)  // expanded ids per routing block
#define ROUTE_CHUNKS (ROUTE_IDS / 64)   // 64-id chunks per routing block

// MXFP8 quantisation of a row-major bf16 tensor, 32-value blocks taken over the
// flat element order (k3_moe_prefill_v4.cu:111-140): sf[i] is the E8M0 scale
// of elements [32 i, 32 i + 32), q the e4m3 payload.
//
// The grid supplies one thread per block, as in the reference launch.  Inside a
// wave the 64 blocks of that wave are processed in four steps of 16 blocks:
// lane l takes 16 bytes at wave offset 1024 j + 16 l, so every load and store
// instruction covers one contiguous 1 KB (512 B for q) and the block amax is a
// quad max.
extern "C" __global__ void __launch_bounds__(256) kern_k3_moe_quant(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ sf,
    int rows, int cols) {
  const long long nblk = (long long)rows * cols / 32;
  const int l = threadIdx.x & 63;
  const long long first = (long long)blockIdx.x * blockDim.x + (threadIdx.x & ~63);
  if (first >= nblk) return;
  k3_u4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // past the end: the last block is re-read, nothing is stored
    const long long blk = min(first + 16 * j + (l >> 2), nblk - 1);
    v[j] = k3_ld16_nt(x + blk * 32 + (l & 3) * 8);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long blk = first + 16 * j + (l >> 2);
    k3_u2 qv;
    const int e = k3_mx_quad(v[j], &qv);  // quad-wide: every lane takes part
    if (blk < nblk) {
      k3_st8_nt(q + blk * 32 + (l & 3) * 8, qv);
      if ((l & 3) == 0) sf[blk] = (uint8_t)(e + 127);
    }
  }
}

// ---------------------------------------------------------------- EP routing
// Local slot of a global expert id, or -1 when another rank owns it
// (k3_moe_prefill_v4.cu:100-109).
K3_DEV int k3_local_expert(int id, int rank, int E) {
#ifdef EP_STRIDED
  if (id % EP_RANKS != rank) return -1;
  const int e = id / EP_RANKS;
  return e < E ? e : -1;
#else
  const int e = id - rank * E;
  return (e >= 0 && e < E) ? e : -1;
#endif
}

// blockcount[b][e]: ids of local expert e among tokens [256 b, 256 b + 256)
// (k3_moe_prefill_v4.cu:142-157).  LDS counters; a count is order-free.
extern "C" __global__ void __launch_bounds__(ROUTE_BLOCK) kern_k3_moe_route_count(
    const int* __restrict__ ids, int T, int rank, int E, int* __restrict__ blockcount) {
  __shared__ int cnt[MAX_E];
  if ((int)threadIdx.x < E) cnt[threadIdx.x] = 0;
  __syncthreads();
  const int t = blockIdx.x * ROUTE_BLOCK + threadIdx.x;
  if (t < T) {
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
      const int e = k3_local_expert(ids[(size_t)t * TOPK + k], rank, E);
      if (e >= 0) atomicAdd(&cnt[e], 1);
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < E) blockcount[blockIdx.x * E + threadIdx.x] = cnt[threadIdx.x];
}

// Wave-wide inclusive prefix sum of integers, GFX9 DPP: row_shr 1, 2, 4, 8 scan
// each 16-lane row (lanes without a source add 0), row_bcast15 carries row 0's
// total into row 1 and row 2's into row 3, row_bcast31 carries rows 0-1 into
// rows 2-3.
K3_DEV int k3_wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, K3_DPP_ROW_BCAST15, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, K3_DPP_ROW_BCAST31, 0xc, 0xf, false);
  return v;
}

// Routing tables (k3_moe_prefill_v4.cu:159-203): count[e] = sum over blocks,
// off = exclusive scan of ceil(count / tile) (CTA units), blockoff[b][e] =
// tile off[e] + the expert's count in blocks before b, padding rows of an
// expert's last tile route token 0, cta_batch / cta_limit per CTA index.
// One workgroup of 16 waves.  The per-block counts are staged in LDS with
// coalesced loads (when blocks * E fits); wave w owns experts w, w + 16, ...
// for the totals, the blockoff scan (64 blocks per DPP scan), the padding rows
// and the expert's CTA range [off[e], off[e+1]); wave 0 scans the CTA units of
// all experts (lane = expert).  Staged blockoff values replace the counts in
// LDS and leave in one coalesced pass.
#define RT_STAGE 8192  // ints of staged per-block counts (32 KB)

extern "C" __global__ void __launch_bounds__(1024) kern_k3_moe_route_tables(
    const int* __restrict__ blockcount, int blocks, int E, int tile, int* __restrict__ blockoff,
    int* __restrict__ cta_batch, int* __restrict__ cta_limit, int* __restrict__ num_non_exiting,
    int* __restrict__ total_padded, int* __restrict__ route_map) {
  __shared__ int bc[RT_STAGE];
  __shared__ int count[MAX_E], off[MAX_E + 1];
#ifdef TILE_SHIFT
  tile = 1 << TILE_SHIFT;
#endif
  if (E < 1 || E > MAX_E) {  // no local experts: nothing routed
    if (threadIdx.x == 0) { num_non_exiting[0] = 0; total_padded[0] = 0; }
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int n = blocks * E;
  const bool staged = n <= RT_STAGE;
  if (staged)
    for (int i = threadIdx.x; i < n; i += blockDim.x) bc[i] = blockcount[i];
  __syncthreads();
  for (int e = wave; e < E; e += nw) {
    int sum = 0;
    for (int b = lane; b < blocks; b += 64) sum += staged ? bc[b * E + e] : blockcount[b * E + e];
    sum = __builtin_amdgcn_readlane(k3_wave_incl_scan(sum), 63);
    if (lane == 0) count[e] = sum;
  }
  __syncthreads();
  if (wave == 0) {
    const int u = lane < E ? (count[lane] + tile - 1) / tile : 0;
    const int incl = k3_wave_incl_scan(u);
    if (lane < E) off[lane] = incl - u;
    if (lane == E - 1) {
      off[E] = incl;
      num_non_exiting[0] = incl;
      total_padded[0] = incl * tile;
    }
  }
  __syncthreads();
  for (int e = wave; e < E; e += nw) {
    int base = off[e] * tile;
    for (int b0 = 0; b0 < blocks; b0 += 64) {
      const int b = b0 + lane;
      const int c = b < blocks ? (staged ? bc[b * E + e] : blockcount[b * E + e]) : 0;
      const int incl = k3_wave_incl_scan(c);
      if (b < blocks) {
        if (staged) bc[b * E + e] = base + incl - c;  // column e is this wave's alone
        else blockoff[b * E + e] = base + incl - c;
      }
      base += __builtin_amdgcn_readlane(incl, 63);
    }
    const int lim = off[e] * tile + count[e];
    for (int r = lim + lane; r < off[e + 1] * tile; r += 64) route_map[r] = 0;
    for (int i = off[e] + lane; i < off[e + 1]; i += 64) {
      cta_batch[i] = e;
      cta_limit[i] = min((i + 1) * tile, lim);
    }
  }
  if (staged) {
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) blockoff[i] = bc[i];
  }
}

// Lanes of the wave holding the same local expert e (0 <= e < 64) as this lane:
// the lanes with e >= 0, narrowed by one ballot per bit of e.  Meaningless for
// lanes with e < 0.
K3_DEV uint64_t k3_expert_peers(int e) {
  uint64_t m = __ballot(e >= 0);
#pragma unroll
  for (int b = 0; b < 6; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t ones = __ballot(bit);
    m &= bit ? ones : ~ones;
  }
  return m;
}

// Route scatter (k3_moe_prefill_v4.cu:205-252).  For the expanded id
// idx = t TOPK + k of routing block b with local expert e, the permuted row is
// blockoff[b][e] + #{idx' < idx in block b with expert e}: a stable counting
// sort of the block's ids by local expert.  The block's ROUTE_IDS ids are cut
// into 64-id chunks in idx order; a lane's rank among the chunk's lanes of its
// expert comes from bit ballots, the chunk's per-expert counts go to LDS, and one
// DPP scan per expert across the chunks (lane = chunk) turns them into each
// chunk's base.  LDS rows are padded to MAX_E + 1 so that scan reads one bank
// per lane.
static_assert(MAX_E <= 64, "expert ids are matched with 6 bit ballots");

extern "C" __global__ void __launch_bounds__(32 * SCATTER_WARPS) kern_k3_moe_route_scatter(
    const int* __restrict__ ids, const int* __restrict__ blockoff, int T, int rank, int E,
    int* __restrict__ route_map, int* __restrict__ exp2perm) {
  __shared__ int hist[ROUTE_CHUNKS][MAX_E + 1];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  constexpr int CPW = (ROUTE_CHUNKS + (32 * SCATTER_WARPS / 64) - 1) / (32 * SCATTER_WARPS / 64);
  const long long base = (long long)blockIdx.x * ROUTE_IDS;
  const long long nid = (long long)T * TOPK;
  for (int i = threadIdx.x; i < ROUTE_CHUNKS * (MAX_E + 1); i += blockDim.x) (&hist[0][0])[i] = 0;
  int ex[CPW];
  long long idx[CPW];
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    idx[r] = base + c * 64 + lane;
    ex[r] = c < ROUTE_CHUNKS && idx[r] < nid ? k3_local_expert(ids[idx[r]], rank, E) : -1;
  }
  __syncthreads();
  int rk[CPW];
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    const uint64_t peers = k3_expert_peers(ex[r]);
    rk[r] = __builtin_popcountll(peers & below);
    if (c < ROUTE_CHUNKS && ex[r] >= 0 && rk[r] == 0) hist[c][ex[r]] = __builtin_popcountll(peers);
  }
  __syncthreads();
  for (int e = wave; e < E; e += nw) {
    int carry = 0;
    for (int c0 = 0; c0 < ROUTE_CHUNKS; c0 += 64) {
      const int c = c0 + lane;
      const int n = c < ROUTE_CHUNKS ? hist[c][e] : 0;
      const int incl = k3_wave_incl_scan(n);
      if (c < ROUTE_CHUNKS) hist[c][e] = carry + incl - n;
      carry += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    if (c >= ROUTE_CHUNKS || idx[r] >= nid) continue;
    const int e = ex[r];
    if (e < 0) { exp2perm[idx[r]] = -1; continue; }
    const int row = blockoff[blockIdx.x * E + e] + hist[c][e] + rk[r];
    route_map[row] = (int)(idx[r] / TOPK);
    exp2perm[idx[r]] = row;
  }
}

// One-launch EP routing (no reference entry; the reference runs the three
// launches above): the same outputs as route_count -> route_tables ->
// route_scatter, the stable counting sort of the expanded ids by local expert
// with 128-row tile padding.
//
//   k3h_moe_route_fused(ids, T, rank, E, blockcount, blockoff, cta_batch,
//       cta_limit, num_non_exiting, total_padded, route_map, exp2perm, sync)
//       grid ceil(T / 256) (at most RF_MAX_BLOCKS), block 32 * SCATTER_WARPS
//
// Workgroup b owns routing block b.  Phase 1 is the scatter's first half: each
// 64-id chunk's per-expert counts and in-chunk ranks (bit ballots), then one
// DPP scan per expert across the chunks, whose carry is the block's count;
// the counts go to blockcount[b].  A grid barrier follows (the grid is at most
// RF_MAX_BLOCKS workgroups, and the host checks that the GPU holds all of them
// at once before it launches): thread 0 of each workgroup adds one to sync[0]
// and waits until it reaches the grid size.  The wait is bounded and all-or-
// nothing: after RF_SPIN_LIMIT polls a workgroup gives up by a compare-and-swap
// that subtracts RF_POISON from the count it last read, which succeeds only if
// no arrival came since, so the count then stays negative and no workgroup can
// pass afterwards; a workgroup that reads a negative count gives up too.  Every
// arrival and the poison act on one word, so either the count reaches the grid
// size (every workgroup passes) or it is poisoned first (none passes).  On
// failure each workgroup writes exp2perm = -1 for its own ids (no slot is
// local, so finalize sums nothing) and workgroup 0 writes num_non_exiting = 0
// and total_padded = -1 (no route tile for the GEMMs or the permute); the other
// tables are left as they were.  Each workgroup then adds one to sync[1]; the
// last to do so puts both words back to 0, so the caller zeroes `sync` once and
// every later launch finds it zeroed, after a failure as well.  Launches that
// share one `sync` must not overlap.
//
// Phase 2 (every workgroup, from the counts of all blocks, read with agent-scope
// loads): per expert the total and this block's prefix over the blocks before
// it, the CTA offsets off = exclusive scan of ceil(total / tile), and then the
// rows route_map[row] = t, exp2perm[t TOPK + k] = row of the block's ids.  The
// table outputs are spread over the workgroups: workgroup b writes blockoff[b],
// and the padding rows and cta_batch / cta_limit of the experts e with
// e % grid == b; workgroup 0 writes num_non_exiting and total_padded.
#define RF_MAX_BLOCKS 256        // T <= 65536 on the one-launch path
#define RF_SPIN_LIMIT (1 << 18)  // polls of the grid barrier before giving up
#define RF_POISON (1 << 20)      // > RF_MAX_BLOCKS: a poisoned count never reaches the grid size
#define RF_GROUPS 16             // block groups of the phase-2 count sums

K3_DEV int rf_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
K3_DEV void rf_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" __global__ void __launch_bounds__(32 * SCATTER_WARPS) k3h_moe_route_fused(
    const int* __restrict__ ids, int T, int rank, int E, int* __restrict__ blockcount,
    int* __restrict__ blockoff, int* __restrict__ cta_batch, int* __restrict__ cta_limit,
    int* __restrict__ num_non_exiting, int* __restrict__ total_padded, int* __restrict__ route_map,
    int* __restrict__ exp2perm, int* __restrict__ sync) {
  __shared__ int hist[ROUTE_CHUNKS][MAX_E + 1];
  __shared__ int pre_s[MAX_E], tot_s[MAX_E], off_s[MAX_E + 1];
  __shared__ int part_s[2][RF_GROUPS][MAX_E];  // [tot | pre][g][e]
  __shared__ int ok_s;
#ifdef TILE_SHIFT
  constexpr int tile = 1 << TILE_SHIFT;
#else
  constexpr int tile = 128;
#endif
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int b = blockIdx.x, nblk = gridDim.x;
  constexpr int CPW = (ROUTE_CHUNKS + (32 * SCATTER_WARPS / 64) - 1) / (32 * SCATTER_WARPS / 64);
  const long long base = (long long)b * ROUTE_IDS;
  const long long nid = (long long)T * TOPK;

  // ---- phase 1: this block's ids, in-chunk ranks, chunk bases, block counts
  for (int i = threadIdx.x; i < ROUTE_CHUNKS * (MAX_E + 1); i += blockDim.x) (&hist[0][0])[i] = 0;
  int ex[CPW];
  long long idx[CPW];
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    idx[r] = base + c * 64 + lane;
    ex[r] = c < ROUTE_CHUNKS && idx[r] < nid ? k3_local_expert(ids[idx[r]], rank, E) : -1;
  }
  __syncthreads();
  int rk[CPW];
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    const uint64_t peers = k3_expert_peers(ex[r]);
    rk[r] = __builtin_popcountll(peers & below);
    if (c < ROUTE_CHUNKS && ex[r] >= 0 && rk[r] == 0) hist[c][ex[r]] = __builtin_popcountll(peers);
  }
  __syncthreads();
  for (int e = wave; e < E; e += nw) {
    int carry = 0;
    for (int c0 = 0; c0 < ROUTE_CHUNKS; c0 += 64) {
      const int c = c0 + lane;
      const int n = c < ROUTE_CHUNKS ? hist[c][e] : 0;
      const int incl = k3_wave_incl_scan(n);
      if (c < ROUTE_CHUNKS) hist[c][e] = carry + incl - n;
      carry += __builtin_amdgcn_readlane(incl, 63);
    }
    // written through to the device's coherence point (system-scope store)
    if (lane == 0) __hip_atomic_store(&blockcount[b * E + e], carry, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }

  // ---- grid barrier (bounded wait), then the reset of `sync` by the last leaver.
  // The counts travel without cache maintenance: they were stored write-through,
  // every wave waits for its stores to complete (vmcnt 0) before the workgroup
  // barrier, so when thread 0 adds its arrival the block's counts are at the
  // coherence point; the arrival counter is polled, and the counts read in phase
  // 2, with agent-coherent loads, which do not return stale L2 lines.  (An
  // agent-scope release / acquire pair, which writes back and invalidates the
  // L2 of every arriving wave, measured 19.1 us against 15.0 us for this.)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(&sync[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int ok = 1, polls = 0, v;
    // Bounded: past the limit each poll ends the loop (count complete, count
    // poisoned, or this poison succeeded) unless an arrival changed the count
    // between the load and the swap, which happens at most nblk times.
    while ((v = rf_load(&sync[0])) < nblk) {
      if (v < 0) { ok = 0; break; }  // another workgroup gave up
      if (++polls > RF_SPIN_LIMIT) {
        if (__hip_atomic_compare_exchange_strong(&sync[0], &v, v - RF_POISON, __ATOMIC_RELAXED,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          ok = 0;
          break;
        }
        continue;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (__hip_atomic_fetch_add(&sync[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblk - 1) {
      rf_store(&sync[0], 0);
      rf_store(&sync[1], 0);
    }
    ok_s = ok;
  }
  __syncthreads();
  if (!ok_s) {  // no workgroup passed the barrier: publish "nothing routed"
#pragma unroll
    for (int r = 0; r < CPW; ++r) {
      const int c = wave + r * nw;
      if (c < ROUTE_CHUNKS && idx[r] < nid) exp2perm[idx[r]] = -1;
    }
    if (b == 0 && threadIdx.x == 0) {
      num_non_exiting[0] = 0;
      total_padded[0] = -1;
    }
    return;
  }

  // ---- phase 2: per-expert totals and this block's prefix, CTA offsets.  Thread
  // (g, e), g < G = min(blockDim / E, RF_GROUPS), sums the counts of expert e over the blocks
  // b' = g (mod G): rows of blockcount are read whole (E consecutive ints per
  // group of threads) and every thread's loads are independent, so the counts
  // arrive in one memory round trip; the G partial sums meet in LDS.
  {
    const int G = min((int)blockDim.x / E, RF_GROUPS);
    const int g = threadIdx.x / E, e = threadIdx.x - g * E;
    int tot = 0, pre = 0;
    if (g < G) {
      for (int bb = g; bb < nblk; bb += G) {
        const int v = rf_load(&blockcount[bb * E + e]);
        tot += v;
        pre += bb < b ? v : 0;
      }
      part_s[0][g][e] = tot;
      part_s[1][g][e] = pre;
    }
    __syncthreads();
    if ((int)threadIdx.x < E) {
      int t = 0, p2 = 0;
      for (int k = 0; k < G; ++k) { t += part_s[0][k][threadIdx.x]; p2 += part_s[1][k][threadIdx.x]; }
      tot_s[threadIdx.x] = t;
      pre_s[threadIdx.x] = p2;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const int u = lane < E ? (tot_s[lane] + tile - 1) / tile : 0;
    const int incl = k3_wave_incl_scan(u);
    if (lane < E) off_s[lane] = incl - u;
    if (lane == E - 1) {
      off_s[E] = incl;
      if (b == 0) {
        num_non_exiting[0] = incl;
        total_padded[0] = incl * tile;
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) blockoff[b * E + e] = off_s[e] * tile + pre_s[e];
  for (int e = b + nblk * wave; e < E; e += nblk * nw) {  // experts owned by this workgroup
    const int lim = off_s[e] * tile + tot_s[e];
    for (int r = lim + lane; r < off_s[e + 1] * tile; r += 64) route_map[r] = 0;
    for (int i = off_s[e] + lane; i < off_s[e + 1]; i += 64) {
      cta_batch[i] = e;
      cta_limit[i] = min((i + 1) * tile, lim);
    }
  }
#pragma unroll
  for (int r = 0; r < CPW; ++r) {
    const int c = wave + r * nw;
    if (c >= ROUTE_CHUNKS || idx[r] >= nid) continue;
    const int e = ex[r];
    if (e < 0) { exp2perm[idx[r]] = -1; continue; }
    const int row = off_s[e] * tile + pre_s[e] + hist[c][e] + rk[r];
    route_map[row] = (int)(idx[r] / TOPK);
    exp2perm[idx[r]] = row;
  }
}

// Weighted finalize (k3_moe_prefill_v4.cu:254-302): out[t, c] = bf16(sum over k
// ascending of wts[t][k] * f32(fc2[exp2perm[t TOPK + k], c])) over the local
// slots, f32 accumulator from 0, one fma per term.  Manifest geometry: grid
// ceil(T / 2), block 128, so each wave owns one token: lanes < TOPK read the
// token's slots and a ballot compacts the local ones (k ascending).
//
// The row is walked in steps of FVN 16-byte vectors per lane.  The number of
// local slots n is uniform over the wave, so the step loop is instantiated per
// n (k3_fin_row<n, FVN>) and contains no branch: vector indices past the row
// are clamped for loads and stores alike (a clamped lane loads, sums and
// stores exactly the bytes of the row's last vector), and the next step's loads
// are issued before this step's stores.  The vector memory counter counts
// stores too, in issue order, so the compiler can then wait for each load
// without draining the stores before it.
#ifndef FIN_NT
#define FIN_NT 1
#endif
// Vectors per lane per step, by number of local slots (n = 1, 2, 3..4, 5..8).
// Wide steps keep 14-28 row loads of one wave in flight; the kernel then runs
// one wave per SIMD (about 280 VGPRs), which on MI355X streams this gather
// faster than narrower steps at two or three waves per SIMD.  7 divides the
// 14 vectors per lane of a 7168-column row.
#ifndef FIN_FV1
#define FIN_FV1 7
#endif
#ifndef FIN_FV2
#define FIN_FV2 7
#endif
#ifndef FIN_FV4
#define FIN_FV4 4
#endif
#ifndef FIN_FV8
#define FIN_FV8 2
#endif

K3_DEV k3_u4 k3_fin_ld(const uint16_t* p) { return FIN_NT ? k3_ld16_nt(p) : k3_ld16(p); }

template <int NS, int FVN>
K3_DEV void k3_fin_row(const uint16_t* __restrict__ fc2, const int* srow, const float* sw,
                       uint16_t* __restrict__ orow, int cols, int lane) {
  const int nvec = cols >> 3;
  const int nsteps = (nvec + 64 * FVN - 1) / (64 * FVN);
  k3_u4 x[NS][FVN];
  auto vec = [&](int step, int c) { return min(step * 64 * FVN + lane + 64 * c, nvec - 1); };
  auto load = [&](int step) {
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int c = 0; c < FVN; ++c) x[i][c] = k3_fin_ld(fc2 + (size_t)srow[i] * cols + (size_t)vec(step, c) * 8);
  };
  auto sum_store = [&](int step, bool prefetch) {
    float acc[FVN][8];
#pragma unroll
    for (int c = 0; c < FVN; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[c][j] = 0.0f;
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int c = 0; c < FVN; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[c][2 * j] = __builtin_fmaf(sw[i], k3_bf_lo(x[i][c][j]), acc[c][2 * j]);
          acc[c][2 * j + 1] = __builtin_fmaf(sw[i], k3_bf_hi(x[i][c][j]), acc[c][2 * j + 1]);
        }
    if (prefetch) load(step + 1);
#pragma unroll
    for (int c = 0; c < FVN; ++c) {
      k3_u4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = k3_pack_bf2(acc[c][2 * j], acc[c][2 * j + 1]);
      k3_st16_nt(orow + (size_t)vec(step, c) * 8, o);
    }
  };
  load(0);
  if (nsteps == 1) {
    sum_store(0, false);
    return;
  }
  // Step 0 is peeled so that the loop is entered, and re-entered, with the same
  // operations in flight (the next step's loads, then this step's stores).
  sum_store(0, true);
  for (int step = 1; step + 1 < nsteps; ++step) sum_store(step, true);
  sum_store(nsteps - 1, false);
}

// More than eight local slots (TOPK 16 only): groups of eight slots per step.
K3_DEV void k3_fin_row_many(const uint16_t* __restrict__ fc2, const int* srow, const float* sw,
                            int n, uint16_t* __restrict__ orow, int cols, int lane) {
  const int nvec = cols >> 3;
  for (int v0 = 0; v0 < nvec; v0 += 64) {
    const int v = min(v0 + lane, nvec - 1);
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int i0 = 0; i0 < n; i0 += 8) {
      k3_u4 x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = k3_fin_ld(fc2 + (size_t)srow[min(i0 + i, n - 1)] * cols + (size_t)v * 8);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i0 + i >= n) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[2 * j] = __builtin_fmaf(sw[i0 + i], k3_bf_lo(x[i][j]), acc[2 * j]);
          acc[2 * j + 1] = __builtin_fmaf(sw[i0 + i], k3_bf_hi(x[i][j]), acc[2 * j + 1]);
        }
      }
    }
    k3_u4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = k3_pack_bf2(acc[2 * j], acc[2 * j + 1]);
    k3_st16_nt(orow + (size_t)v * 8, o);
  }
}

// Typed-call finalize (no reference entry; the same bits as kern_k3_moe_finalize):
//   k3h_moe_finalize_rows(fc2, exp2perm, wts, out, T, cols)
//       grid T, block 64 * FIN_NW
// One workgroup per token.  Thread i of the workgroup handles the row's vectors
// i + 64 FIN_NW j, j < FIN_J, of every local slot: all of them are loaded before
// the first sum, so a token's whole gather is in flight at once, spread over
// FIN_NW waves of few registers each (about 75 VGPRs, six waves per SIMD),
// instead of one wave of about 280 VGPRs walking the row in steps (one wave per
// SIMD).  Each wave reads the token's slots itself.  Measured on MI355X at
// config 5 (16384 tokens, 7168 columns): 7 waves per token 120.3 us against
// 125.8 us for the manifest entry (clean caches); 2 / 4 / 14 waves 122.0 /
// 120.8 / 131.6 us; 2, 4 or 8 tokens per workgroup taken in turn with their
// slots fetched in one load, 123.2 / 129.0 / 137.1 us.
#ifndef FIN_NW
#define FIN_NW 7
#endif
#define FIN_NT_THREADS (64 * FIN_NW)
#define FIN_J ((7168 / 8 + FIN_NT_THREADS - 1) / FIN_NT_THREADS)  // vectors per thread at 7168 columns

template <int NS>
K3_DEV void k3_fin_tok(const uint16_t* __restrict__ fc2, const int* srow, const float* sw,
                       uint16_t* __restrict__ orow, int cols, int tid) {
  const int nvec = cols >> 3;
  // rows wider than FIN_J vectors per thread take several chunks
  for (int v0 = 0; v0 < nvec; v0 += FIN_J * FIN_NT_THREADS) {
    k3_u4 x[NS][FIN_J];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int j = 0; j < FIN_J; ++j) {
        const int v = min(v0 + tid + FIN_NT_THREADS * j, nvec - 1);
        x[i][j] = k3_fin_ld(fc2 + (size_t)srow[i] * cols + (size_t)v * 8);
      }
#pragma unroll
    for (int j = 0; j < FIN_J; ++j) {
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = __builtin_fmaf(sw[i], k3_bf_lo(x[i][j][q]), acc[2 * q]);
          acc[2 * q + 1] = __builtin_fmaf(sw[i], k3_bf_hi(x[i][j][q]), acc[2 * q + 1]);
        }
      k3_u4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = k3_pack_bf2(acc[2 * q], acc[2 * q + 1]);
      // a clamped thread stores the same bytes as the thread owning the last vector
      k3_st16_nt(orow + (size_t)min(v0 + tid + FIN_NT_THREADS * j, nvec - 1) * 8, o);
    }
  }
}

extern "C" __global__ void __launch_bounds__(FIN_NT_THREADS) k3h_moe_finalize_rows(
    const uint16_t* __restrict__ fc2, const int* __restrict__ exp2perm,
    const float* __restrict__ wts, uint16_t* __restrict__ out, int T, int cols) {
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const int t = blockIdx.x;
  if (t >= T || cols < 8) return;
  int p = -1;
  float w = 0.0f;
  if (lane < TOPK) {
    p = exp2perm[(size_t)t * TOPK + lane];
    w = wts[(size_t)t * TOPK + lane];
  }
  const uint64_t live = __ballot(p >= 0);
  const int n = __builtin_popcountll(live);
  int srow[TOPK];
  float sw[TOPK];
  {
    uint64_t m = live;
#pragma unroll
    for (int i = 0; i < TOPK; ++i) {
      const int k = m ? __builtin_ctzll(m) : 0;
      srow[i] = __builtin_amdgcn_readfirstlane(__shfl(p, k, 64));
      sw[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__shfl(w, k, 64))));
      m &= m - 1;
    }
  }
  uint16_t* __restrict__ orow = out + (size_t)t * cols;
  switch (n) {
    case 0: {  // no local slot: the row is bf16(0)
      const k3_u4 z = {0u, 0u, 0u, 0u};
      for (int v = tid; v < (cols >> 3); v += FIN_NT_THREADS) k3_st16_nt(orow + (size_t)v * 8, z);
      break;
    }
    case 1: k3_fin_tok<1>(fc2, srow, sw, orow, cols, tid); break;
    case 2: k3_fin_tok<2>(fc2, srow, sw, orow, cols, tid); break;
    case 3: k3_fin_tok<3>(fc2, srow, sw, orow, cols, tid); break;
    case 4: k3_fin_tok<4>(fc2, srow, sw, orow, cols, tid); break;
    case 5: k3_fin_tok<5>(fc2, srow, sw, orow, cols, tid); break;
    case 6: k3_fin_tok<6>(fc2, srow, sw, orow, cols, tid); break;
    case 7: k3_fin_tok<7>(fc2, srow, sw, orow, cols, tid); break;
    case 8: k3_fin_tok<8>(fc2, srow, sw, orow, cols, tid); break;
    default: {  // more than eight local slots (TOPK 16): eight at a time per vector
      for (int v = tid; v < (cols >> 3); v += FIN_NT_THREADS) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
        for (int i0 = 0; i0 < n; i0 += 8) {
          k3_u4 x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = k3_fin_ld(fc2 + (size_t)srow[min(i0 + i, n - 1)] * cols + (size_t)v * 8);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (i0 + i >= n) break;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc[2 * q] = __builtin_fmaf(sw[i0 + i], k3_bf_lo(x[i][q]), acc[2 * q]);
              acc[2 * q + 1] = __builtin_fmaf(sw[i0 + i], k3_bf_hi(x[i][q]), acc[2 * q + 1]);
            }
          }
        }
        k3_u4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = k3_pack_bf2(acc[2 * q], acc[2 * q + 1]);
        k3_st16_nt(orow + (size_t)v * 8, o);
      }
      break;
    }
  }
}

extern "C" __global__ void __launch_bounds__(128) kern_k3_moe_finalize(
    const uint16_t* __restrict__ fc2, const int* __restrict__ exp2perm,
    const float* __restrict__ wts, uint16_t* __restrict__ out, int T, int cols) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 2 + (threadIdx.x >> 6);
  if (t >= T || cols < 8) return;
  int p = -1;
  float w = 0.0f;
  if (lane < TOPK) {
    p = exp2perm[(size_t)t * TOPK + lane];
    w = wts[(size_t)t * TOPK + lane];
  }
  const uint64_t live = __ballot(p >= 0);
  const int n = __builtin_popcountll(live);
  int srow[TOPK];
  float sw[TOPK];
  {
    uint64_t m = live;
#pragma unroll
    for (int i = 0; i < TOPK; ++i) {
      const int k = m ? __builtin_ctzll(m) : 0;
      srow[i] = __builtin_amdgcn_readfirstlane(__shfl(p, k, 64));
      sw[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__shfl(w, k, 64))));
      m &= m - 1;
    }
  }
  uint16_t* __restrict__ orow = out + (size_t)t * cols;
  switch (n) {
    case 0: {  // no local slot: the row is bf16(0)
      const k3_u4 z = {0u, 0u, 0u, 0u};
      for (int v = lane; v < (cols >> 3); v += 64) k3_st16_nt(orow + (size_t)v * 8, z);
      break;
    }
    case 1: k3_fin_row<1, FIN_FV1>(fc2, srow, sw, orow, cols, lane); break;
    case 2: k3_fin_row<2, FIN_FV2>(fc2, srow, sw, orow, cols, lane); break;
    case 3: k3_fin_row<3, FIN_FV4>(fc2, srow, sw, orow, cols, lane); break;
    case 4: k3_fin_row<4, FIN_FV4>(fc2, srow, sw, orow, cols, lane); break;
    case 5: k3_fin_row<5, FIN_FV8>(fc2, srow, sw, orow, cols, lane); break;
    case 6: k3_fin_row<6, FIN_FV8>(fc2, srow, sw, orow, cols, lane); break;
    case 7: k3_fin_row<7, FIN_FV8>(fc2, srow, sw, orow, cols, lane); break;
    case 8: k3_fin_row<8, FIN_FV8>(fc2, srow, sw, orow, cols, lane); break;
    default: k3_fin_row_many(fc2, srow, sw, n, orow, cols, lane); break;
  }
}

// MXFP8 permute: rows of the token-major MXFP8 activation gathered into the
// expert-contiguous order of route_map (padding rows carry token 0, as routed).
// One row per wave (r = global wave id, striding by the grid's waves), rows
// r >= *total_padded exit; all of a row's loads are issued before its stores.
// Per row cols payload bytes (NV = cols / 1024 16-byte vectors per lane, a
// template parameter so that no load is predicated) and cols / 32 scale bytes
// (up to two words per lane; lanes past the row's words re-read its last word
// and do not store).  cols % 1024 == 0, cols <= 16384.
template <int NV>
K3_DEV void k3_permute_row(const uint8_t* __restrict__ q, const uint8_t* __restrict__ sf,
                           int t, int r, int cols, uint8_t* __restrict__ pq,
                           uint8_t* __restrict__ psf, int lane) {
  const int sfw = cols >> 7;  // scale words per row: up to 128, two per lane
  // cacheable loads: a token's row is read once per local expert it routes to
  // (about 2.2 times at top-8 over 56 of 224 experts), far apart in route_map's
  // expert order, and the whole q (117 MB at 16384 x 7168) stays in the 256 MB
  // MALL between them (measured: 90.5 -> 75.8 us after a clean flush, 85.1 ->
  // 74.3 us back to back over four rotating input / output sets, identical
  // outputs; 89.5 -> 96 us after a dirty flush, whose lines the loads evict)
  k3_u4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = k3_ld16(q + (size_t)t * cols + (size_t)(lane + 64 * j) * 16);
  const uint32_t* srow = (const uint32_t*)(sf + (size_t)t * (cols >> 5));
  const uint32_t sw0 = srow[min(lane, sfw - 1)], sw1 = srow[min(lane + 64, sfw - 1)];
#pragma unroll
  for (int j = 0; j < NV; ++j) k3_st16_nt(pq + (size_t)r * cols + (size_t)(lane + 64 * j) * 16, v[j]);
  uint32_t* drow = (uint32_t*)(psf + (size_t)r * (cols >> 5));
  if (lane < sfw) drow[lane] = sw0;
  if (lane + 64 < sfw) drow[lane + 64] = sw1;
}

extern "C" __global__ void __launch_bounds__(256) k3h_moe_permute_mx(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ sf, const int* __restrict__ route_map,
    const int* __restrict__ total_padded, int max_rows, int cols, uint8_t* __restrict__ pq,
    uint8_t* __restrict__ psf) {
  const int lane = threadIdx.x & 63;
  const int nrows = min(total_padded[0], max_rows);  // pq / psf hold max_rows rows
  const int nwaves = gridDim.x * (blockDim.x >> 6);
  for (int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < nrows; r += nwaves) {
    const int t = route_map[r];
    switch (cols >> 10) {
#define K3_PM_CASE(n) \
  case n: k3_permute_row<n>(q, sf, t, r, cols, pq, psf, lane); break;
      K3_PM_CASE(1) K3_PM_CASE(2) K3_PM_CASE(3) K3_PM_CASE(4)
      K3_PM_CASE(5) K3_PM_CASE(6) K3_PM_CASE(7) K3_PM_CASE(8)
      K3_PM_CASE(9) K3_PM_CASE(10) K3_PM_CASE(11) K3_PM_CASE(12)
      K3_PM_CASE(13) K3_PM_CASE(14) K3_PM_CASE(15) K3_PM_CASE(16)
#undef K3_PM_CASE
      default: break;
    }
  }
}

// Load-time weight layouts (k3_moe_prefill_v4.cu:69-80, 304-327): row r of each
// expert's destination takes source row shuffle(r); scales also re-laid in
// 128 x 4 blocks.
K3_DEV int k3_w_shuffle_row(int r, int n, int gated) {
  const int u = (r / 32) * 32 + (r % 8) * 4 + (r % 32) / 8;
  return gated ? (u % 2 ? n / 2 : 0) + u / 2 : u;
}

extern "C" __global__ void __launch_bounds__(256) kern_k3_moe_w_shuffle(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int experts, int n, int row_bytes,
    int gated) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = row_bytes / 16;
  if (i >= (long long)experts * n * per_row) return;
  const int c = (int)(i % per_row), r = (int)(i / per_row % n), e = (int)(i / per_row / n);
  k3_st16(dst + i * 16, k3_ld16(src + ((long long)e * n + k3_w_shuffle_row(r, n, gated)) * row_bytes + (long long)c * 16));
}

extern "C" __global__ void __launch_bounds__(256) kern_k3_moe_sf_shuffle(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int experts, int n, int kg,
    int gated) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)experts * n * kg) return;
  const int c = (int)(i % kg), r = (int)(i / kg % n), e = (int)(i / kg / n);
  const long long at = ((long long)(r / 128) * (kg / 4) + c / 4) * 512 + (r % 32) * 16 +
                       ((r % 128) / 32) * 4 + c % 4;
  dst[(long long)e * n * kg + at] = src[((long long)e * n + k3_w_shuffle_row(r, n, gated)) * kg + c];
}
