// Epoch / arrival barrier of the TP collectives over peer pointers.  One source,
// three module keys, every one exporting the same entries:
//
//   k3_collectives (the barrier entries of k3_collectives.cu; its all-gather and
//   reduce-scatter data kernels move bytes between GPUs and are not built here,
//   so a lookup of them reports a missing entry):
//     kern_k3_flags_init(flags, n)         any grid: flags[0 .. n) = 0
//     kern_k3_epoch_bump(flags)            flags[0] += gridDim.x, once per launch
//   k3_rs_arrive1 / k3_rs_arrive_v2 (k3_rs_arrive1.cu, k3_rs_arrive_v2.cu):
//     kern_k3_rs_arrive1(src, dst, src_peer, flags, flags_peer, count, units,
//                        slot, order, rank, nranks)          grid 1, block 32 or 64
//   and, with no counterpart in the reference:
//     k3h_rs_arrive_mask(flags, flags_peer, units, slot, nranks, missing)
//                                          the same barrier, reporting the peers
//                                          whose counters missed the target
//
// Protocol (k3_collectives.cu:21-35).  `flags` is this rank's array of u64
// counters, `flags_peer[q]` the device address of rank q's copy of it (rank
// `rank` itself included).  flags[0] is the epoch: every program call first adds
// the number of arrivals its collectives will produce (the collective grid,
// 896 at 16,384 tokens), so after the i-th call it is the total over calls
// 1..i.  A collective on slot s adds its arrivals to this rank's flags[s], then
// waits until every rank's flags[s] has reached this rank's flags[0].  Counters
// are never reset: a counter left at an earlier call's total is below every
// later target, since each call adds at least one arrival.  All counters stay
// far below 2^32, so the low word of a u64 (little-endian: its first 4 bytes)
// is compared, as the reference does.
//
// The arrival is one workgroup adding the whole grid's units in one atomic
// (k3_rs_arrive_v2.cu:1-29): it runs after this rank's producer kernel on the
// same stream, so the counter moves only once the producer's stores are done.
// Lane q < nranks polls rank q's counter (the polls of the peers overlap instead
// of running one after another, k3_rs_arrive_v2.cu:56-62).  Ordering:
//   * a system-scope release fence before the add makes this rank's earlier
//     stores (the producer's pushes into peer memory) visible to every agent
//     before any peer can see the arrival;
//   * the add and the polls are system-scope atomics (no stale cached copy of a
//     peer's counter is ever read);
//   * a system-scope acquire fence after the wait orders every later read of
//     peer data after the observed arrivals.
// The wait is bounded: a lane gives up once K3_SPIN_US microseconds of the
// device's constant 100 MHz real-time clock have passed since it started
// polling (default 2 s, the reference's bail-out, K3_SPIN_NS at
// k3_collectives.cu:50, so a dead peer cannot wedge the GPU); between polls a
// lane sleeps for s_sleep 2 (about 128 clocks).
#include "../common/k3_dev.h"

#ifndef K3_SPIN_US
#define K3_SPIN_US 2000000
#endif
#define K3_MAX_RANKS 8
#define K3_RTC_PER_US 100ull  // s_memrealtime ticks per microsecond (100 MHz)

typedef unsigned long long k3_u64;

extern "C" __global__ void __launch_bounds__(256) kern_k3_flags_init(k3_u64* __restrict__ flags,
                                                                    int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    flags[i] = 0ull;
}

extern "C" __global__ void __launch_bounds__(1024) kern_k3_epoch_bump(k3_u64* __restrict__ flags) {
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_add(&flags[0], (k3_u64)gridDim.x, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// The barrier of one rank: add `units` to flags[slot], wait for every rank's
// flags[slot] to reach flags[0].  Returns (in every lane) the mask of ranks q <
// nranks whose counter was still below the target when the lane polling it gave
// up; 0 when every rank arrived.
K3_DEV unsigned k3_rs_arrive(k3_u64* flags, const k3_u64* flags_peer, int units, int slot,
                             int nranks) {
  const int nr = nranks < K3_MAX_RANKS ? nranks : K3_MAX_RANKS;
  const int q = threadIdx.x;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");  // system scope: L2 write-back
  __builtin_amdgcn_s_waitcnt(0);                  // ... completed before the add
  if (q == 0)
    __hip_atomic_fetch_add(&flags[slot], (k3_u64)units, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
  bool missed = false;
  if (q < nr) {
    const uint32_t target = (uint32_t)__hip_atomic_load(&flags[0], __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_SYSTEM);
    typedef __attribute__((address_space(1))) const uint32_t k3_gcu32;
    k3_gcu32* f = (k3_gcu32*)(uintptr_t)(flags_peer[q] + (k3_u64)slot * 8ull);
    const k3_u64 t0 = __builtin_amdgcn_s_memrealtime();
    const k3_u64 limit = (k3_u64)K3_SPIN_US * K3_RTC_PER_US;
    while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) < target) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > limit) {
        missed = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  const unsigned mask = (unsigned)__builtin_amdgcn_ballot_w64(missed);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");  // system scope
  return mask;
}

// kern_k3_rs_arrive1 (k3_rs_arrive1.cu:41, k3_rs_arrive_v2.cu:41): the manifest
// entry.  src, dst, src_peer, count, order and rank are not read (the reference
// takes them so that the arrival shares the collective's argument list).
extern "C" __global__ void __launch_bounds__(64) kern_k3_rs_arrive1(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
    const k3_u64* __restrict__ src_peer, k3_u64* __restrict__ flags,
    const k3_u64* __restrict__ flags_peer, long long count, int units, int slot, int order,
    int rank, int nranks) {
  (void)src; (void)dst; (void)src_peer; (void)count; (void)order; (void)rank;
  k3_rs_arrive(flags, flags_peer, units, slot, nranks);
}

// The same barrier with its outcome: missing[0] = mask of the ranks that had not
// arrived when the wait gave up (bit q for rank q; 0 = all arrived).
extern "C" __global__ void __launch_bounds__(64) k3h_rs_arrive_mask(
    k3_u64* __restrict__ flags, const k3_u64* __restrict__ flags_peer, int units, int slot,
    int nranks, uint32_t* __restrict__ missing) {
  const unsigned mask = k3_rs_arrive(flags, flags_peer, units, slot, nranks);
  if (threadIdx.x == 0) missing[0] = mask;
}
