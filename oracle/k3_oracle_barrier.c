/* CPU oracle: the epoch / arrival barrier of the TP collectives, restated for
 * host threads (each thread plays one rank; its counters are a u64 array in
 * host memory, its peers' arrays are reached through their addresses).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by the tests, never by the product path.
 *
 * Protocol (k3_collectives.cu:21-35): flags[0] is the epoch, raised once per
 * program call by the number of arrivals the call's collectives will add per
 * slot; a collective on slot s adds its arrivals to this rank's flags[s] and
 * waits until every rank's flags[s] has reached this rank's flags[0].  Counters
 * are never reset (k3_collectives.cu:27-35); the comparison is on the low 32
 * bits (k3_rs_arrive1.cu:56-58).
 */
#include <sched.h>
#include <stdint.h>
#include <time.h>

#include "k3_oracle.h"

#define K3O_MAX_RANKS 8

static long long k3o_now_ns(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (long long)ts.tv_sec * 1000000000LL + ts.tv_nsec;
}

/* kern_k3_flags_init (k3_collectives.cu:64-69). */
void k3o_flags_init(uint64_t* flags, int n) {
  for (int i = 0; i < n; ++i) __atomic_store_n(&flags[i], 0ull, __ATOMIC_SEQ_CST);
}

/* kern_k3_epoch_bump (k3_collectives.cu:71-79): one add of the launch's grid size. */
void k3o_epoch_bump(uint64_t* flags, int units) {
  __atomic_fetch_add(&flags[0], (uint64_t)units, __ATOMIC_SEQ_CST);
}

/* kern_k3_rs_arrive1 (k3_rs_arrive1.cu:41-73; k3_rs_arrive_v2.cu:41-76): fence,
 * flags[slot] += units, then for each rank q < min(nranks, 8) wait until the low
 * 32 bits of rank q's flags[slot] (at address flags_peer[q] + 8 slot) reach the
 * low 32 bits of flags[0].  One deadline for the whole wait, spin_ns after it
 * starts (the reference's K3_SPIN_NS bail-out): a rank still below the target at
 * the deadline is given up on.  Returns the mask of the ranks given up on. */
unsigned k3o_rs_arrive(uint64_t* flags, const uint64_t* flags_peer, int units, int slot,
                       int nranks, long long spin_ns) {
  const int nr = nranks < K3O_MAX_RANKS ? nranks : K3O_MAX_RANKS;
  __atomic_thread_fence(__ATOMIC_SEQ_CST);
  __atomic_fetch_add(&flags[slot], (uint64_t)units, __ATOMIC_SEQ_CST);
  const uint32_t target = (uint32_t)__atomic_load_n(&flags[0], __ATOMIC_SEQ_CST);
  const long long t0 = k3o_now_ns();
  unsigned missing = 0;
  for (int q = 0; q < nr; ++q) {
    const uint64_t* f = (const uint64_t*)(uintptr_t)(flags_peer[q] + 8ull * (uint64_t)slot);
    while ((uint32_t)__atomic_load_n(f, __ATOMIC_SEQ_CST) < target) {
      if (k3o_now_ns() - t0 > spin_ns) {
        missing |= 1u << q;
        break;
      }
      sched_yield();
    }
  }
  __atomic_thread_fence(__ATOMIC_SEQ_CST);
  return missing;
}
