// Cross-workgroup exchange inside one launch, for grids that are resident on
// the device all at once (the host sizes them by occupancy).
//
// Values travel through 64-bit slots written by agent-scope relaxed atomic
// stores and polled by agent-scope atomic loads, one value per slot, encoded
// so that no value encodes to zero: a zero word is an empty slot, so every
// slot is its own ready flag and no fence is needed (on gfx950 an agent-scope
// release compiles to a write-back of the whole L2).  Each workgroup empties
// the slots it will fill and then arrives at a start barrier (res_arrive);
// slots are read only after the barrier is complete, so no reader sees what
// a slot held before the call.  Waits are bounded: a slot still empty after
// the launch's poll limit reads as NaN and raises the device's wait-status
// word; the kernels then write NaN over their outputs or skip their writes.
#pragma once

#include <atomic>

#include "common.hpp"

namespace ppo {

constexpr uint64_t kSlotTag = 0x7FF4A5A55A5A0F0FULL;  // a signalling-NaN pattern
constexpr long kSlotSpin = 1L << 22;                  // polls before giving up (default)

// Bounded-wait control of one launch: the poll limit of every wait and the
// current device's wait-status word (library-owned, see wait_ctl).
struct WaitCtl {
  unsigned* status;
  long spin;
};

// Host: fills `w` for a launch on the current device (abi.hip).  Returns a
// PPO code.
int wait_ctl(WaitCtl& w);

// Host: zeroes the allocation-free entry point's scratch on the current
// device, on `stream` (loss.hip).  A wait that gave up can leave arrival
// tags and counters that a later call on the same memory would take for its
// own; ppo_wait_status clears that memory when it reports a give-up.
int scratch_clear(hipStream_t stream);
// The start barrier counts arrivals on kSyncCounters counters, kSyncStride
// words (256 bytes) apart: atomics on one address are serialised by the
// memory (measured ~35 ns each on MI355X, so 1024 arrivals on one counter
// took ~37 us), on separate lines they proceed in parallel.
constexpr int kSyncCounters = 8;
constexpr size_t kSyncStride = 32;
constexpr size_t kSyncWords = kSyncCounters * kSyncStride;  // the barrier's block of words

__device__ __forceinline__ void slot_put(uint64_t* p, double x) {
  uint64_t b = __builtin_bit_cast(uint64_t, x);
  if (x != x) b = 0x7FF8000000000000ULL;  // one NaN pattern, never the tag
  __hip_atomic_store(p, b ^ kSlotTag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double slot_value(uint64_t w) {
  return __builtin_bit_cast(double, w ^ kSlotTag);
}

__device__ __forceinline__ uint64_t slot_peek(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls slot `p` up to `spin` times; a slot still empty then reads as NaN
// and sets `fail` (spin 0: gives up at once).
__device__ __forceinline__ double slot_get(uint64_t* p, long spin, int& fail) {
  for (long it = 0; it < spin; ++it) {
    const uint64_t w = slot_peek(p);
    if (w != 0) return slot_value(w);
    __builtin_amdgcn_s_sleep(1);
  }
  fail = 1;
  return __builtin_nan("");
}

// A word already read (w) or, when it was still empty, the polled value.
__device__ __forceinline__ double slot_or_get(uint64_t w, uint64_t* p, long spin, int& fail) {
  return w ? slot_value(w) : slot_get(p, spin, fail);
}

// Raises the device's wait-status word (one vector atomic; failure path only).
__device__ __forceinline__ void wait_report(unsigned* status) {
  __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void slot_clear(uint64_t* p) {
  __hip_atomic_store(p, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Start barrier: workgroup b arrives on counter b % kSyncCounters, a word
// (nonce:32, count:32).  A workgroup arrives by one compare-and-swap attempt
// that resets a counter tagged with another nonce (an earlier call's, or
// whatever the workspace held) or holding a complete count (a previous replay
// of the same captured call) to (nonce, 0), then one atomic add; neither
// result is waited for, and both go to the same address, so they apply in
// order.  (A retry loop of compare-and-swaps serialises at memory latency.)
// Counter i is complete at (nonce, >= its share of the grid); the barrier is
// complete when every counter is.  `v` is the counter as read after the
// workgroup's slots were emptied.
__device__ inline unsigned sync_share(int i, unsigned nblocks) {
  return (nblocks + kSyncCounters - 1 - i) / kSyncCounters;  // blocks b with b % K == i
}

__device__ inline void res_arrive(uint64_t* ctr, uint64_t v, unsigned nonce, unsigned share) {
  const uint64_t tag = (uint64_t)nonce << 32;
  if ((v >> 32) != nonce || (unsigned)v >= share)
    __hip_atomic_compare_exchange_strong(ctr, &v, tag, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(ctr, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits (at most `spin` polls) until every counter of the barrier at `sync`
// is complete; false when it gave up.  (All counters are read together, so a
// complete barrier costs one round trip.)
__device__ inline bool res_wait(uint64_t* sync, unsigned nonce, unsigned nblocks, long spin) {
  for (long it = 0; it < spin; ++it) {
    uint64_t v[kSyncCounters];
#pragma unroll
    for (int i = 0; i < kSyncCounters; ++i) v[i] = slot_peek(sync + i * kSyncStride);
    bool done = true;
#pragma unroll
    for (int i = 0; i < kSyncCounters; ++i)
      done = done && (i >= (int)nblocks ||
                      ((v[i] >> 32) == nonce && (unsigned)v[i] >= sync_share(i, nblocks)));
    if (done) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Called by wave 0 of every workgroup at its start: empties the `n` slots at
// `mine` (lane-strided), waits until those stores are done, and arrives.
__device__ inline void sync_start(uint64_t* sync, uint64_t* mine, int n, unsigned nonce) {
  const int lane = threadIdx.x % kWave;
  const int i = (int)(blockIdx.x % kSyncCounters);
  uint64_t* ctr = sync + i * kSyncStride;
  for (int q = lane; q < n; q += kWave) slot_clear(mine + q);
  uint64_t v = 0;
  if (lane == 0) v = slot_peek(ctr);
  __builtin_amdgcn_s_waitcnt(0);  // the emptying stores (and that read) are done
  if (lane == 0) res_arrive(ctr, v, nonce, sync_share(i, gridDim.x));
}

// The tag of a launch's barrier counters: the host's nonce mixed with a call
// counter kept in the workspace (`epoch`, any start value).  Every workgroup
// reads the counter before it arrives at the start barrier, and workgroup 0
// advances it (epoch_advance) once that barrier is complete, so a replay of a
// captured launch, which repeats the host's nonce, still gets a tag of its
// own: counters that the previous replay left complete cannot release this
// replay's waiters early.  `e` receives the counter for epoch_advance.
__device__ inline unsigned launch_tag(const uint64_t* epoch, unsigned nonce, uint64_t& e) {
  e = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return nonce ^ (unsigned)((e * 0x9E3779B97F4A7C15ULL) >> 32);
}

__device__ inline void epoch_advance(uint64_t* epoch, uint64_t e) {
  __hip_atomic_store(epoch, e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A different tag for every launch (zero is skipped).
inline unsigned next_nonce() {
  static std::atomic<unsigned> calls{0x5bd1e995u};
  unsigned nonce;
  do {
    nonce = calls.fetch_add(0x9e3779b9u, std::memory_order_relaxed);
  } while (nonce == 0u);
  return nonce;
}

}  // namespace ppo
