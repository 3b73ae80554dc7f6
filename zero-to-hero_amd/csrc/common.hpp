// Shared device/host helpers for libppo_amd (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <tuple>

#include "ppo_amd.h"

namespace ppo {

constexpr int kWave = 64;
constexpr int kBlock = 256;              // threads per workgroup for streaming kernels
constexpr size_t kHeaderBytes = 256;     // WsHeader at the front of every workspace

// Workspace header.  No cross-workgroup combine here uses a release fence: on
// gfx950 an agent-scope release compiles to a full L2 write-back (buffer_wbl2)
// per workgroup.  Values that cross workgroups inside a launch travel through
// agent-scope atomic stores and loads whose completion is awaited explicitly.
struct WsHeader {
  float stats[4];         // {mean, std, denom, 0} written by the stats finaliser
  uint64_t epoch;         // call counter (any start value): Gaussian loss tags, barrier tags
};
static_assert(sizeof(WsHeader) <= kHeaderBytes, "header too big");

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline int hip_status(hipError_t e) { return e == hipSuccess ? PPO_OK : PPO_ERR_HIP_BASE + (int)e; }

// Launch-error check after a hipLaunchKernelGGL.
inline int last_launch_status() { return hip_status(hipGetLastError()); }

// DPP lane move of a double (two 32-bit halves), every lane and bank enabled.
template <int kCtrl>
__device__ __forceinline__ double dpp_move(double x) {
  const int2 v = __builtin_bit_cast(int2, x);
  int2 r;
  r.x = __builtin_amdgcn_update_dpp(0, v.x, kCtrl, 0xF, 0xF, false);
  r.y = __builtin_amdgcn_update_dpp(0, v.y, kCtrl, 0xF, 0xF, false);
  return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ double read_lane(double x, int lane) {
  const int2 v = __builtin_bit_cast(int2, x);
  int2 r;
  r.x = __builtin_amdgcn_readlane(v.x, lane);
  r.y = __builtin_amdgcn_readlane(v.y, lane);
  return __builtin_bit_cast(double, r);
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations (lgkmcnt) but leaves its global loads and stores in flight,
// where __syncthreads() would wait for all of them.  For phases that
// communicate through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave-wide sum, the same value in every lane.  Within each 16-lane row, DPP
// moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror) leave the row's sum in every lane of the row; the four row sums
// are then read out with readlane and added as (r0 + r1) + (r2 + r3).  DPP
// moves are VALU operations; a __shfl_xor butterfly goes through the LDS
// crossbar (ds_bpermute, twice per double) at LDS latency per step.  The
// summation order is fixed, so results are deterministic.
__device__ __forceinline__ double wave_sum(double x) {
  x += dpp_move<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_move<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_move<0x141>(x);  // row_half_mirror
  x += dpp_move<0x140>(x);  // row_mirror
  return (read_lane(x, 0) + read_lane(x, 16)) + (read_lane(x, 32) + read_lane(x, 48));
}

// Block-wide sum of K doubles per thread (whole waves, at most 16); result
// valid in every lane of wave 0.  Each wave reduces its values with wave_sum, and wave 0
// then reduces the per-wave sums the same way (lanes past the last wave add
// zeros), so the order is fixed and no thread loops over the waves.
template <int K>
__device__ inline void block_sum(double (&x)[K]) {
  __shared__ double s_part[16][K];
#pragma unroll
  for (int k = 0; k < K; ++k) x[k] = wave_sum(x[k]);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) s_part[wid][k] = x[k];
  }
  __syncthreads();
  if (wid == 0) {
    const int nw = blockDim.x / kWave;
    double v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = lane < nw ? s_part[lane < 16 ? lane : 0][k] : 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) x[k] = wave_sum(v[k]);
  }
  __syncthreads();
}

// block_sum with LDS-only barriers (lds_barrier): the same fixed order and
// result, but a wave's outstanding global stores are not drained at the
// barriers, as __syncthreads() would do.
template <int K>
__device__ inline void block_sum_lds(double (&x)[K]) {
  __shared__ double s_part[16][K];
#pragma unroll
  for (int k = 0; k < K; ++k) x[k] = wave_sum(x[k]);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) s_part[wid][k] = x[k];
  }
  lds_barrier();
  if (wid == 0) {
    const int nw = blockDim.x / kWave;
    double v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = lane < nw ? s_part[lane < 16 ? lane : 0][k] : 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) x[k] = wave_sum(v[k]);
  }
  lds_barrier();
}

// Sums of `count` partial (n, sum x, sum x^2, pad) quadruples, combined by
// one block in a fixed order (thread t takes partials t, t + blockDim, ...,
// then the block tree), so every call gets bit-identical totals.  Result
// valid in thread 0.
__device__ inline void sum_partials(const double* part, long count, double (&tot)[3]) {
  tot[0] = tot[1] = tot[2] = 0.0;
  // two partials per thread per round, all loads in flight together
  for (long i = threadIdx.x; i < count; i += 2 * blockDim.x) {
    const long j = i + blockDim.x < count ? i + blockDim.x : i;
    const double a0 = part[4 * i + 0], a1 = part[4 * i + 1], a2 = part[4 * i + 2];
    const double b0 = part[4 * j + 0], b1 = part[4 * j + 1], b2 = part[4 * j + 2];
    const bool second = j != i;
    tot[0] += a0;
    tot[1] += a1;
    tot[2] += a2;
    tot[0] += second ? b0 : 0.0;
    tot[1] += second ? b1 : 0.0;
    tot[2] += second ? b2 : 0.0;
  }
  block_sum<3>(tot);
}

// Threads of the one-block finaliser kernels: a whole CU's worth of waves, so
// that the partial loads and the wave reductions run 16 waves wide.
constexpr int kFinalBlock = 1024;

__host__ __device__ inline unsigned int pow2_ceil(unsigned int x) {
  unsigned int p = 1;
  while (p < x) p <<= 1;
  return p;
}

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Workgroups of `kernel` that fit on the current device at once (all CUs),
// for persistent-style grids that loop over tiles.  Falls back to `fallback`
// if the runtime cannot answer.
// The answer is cached per (device, kernel, block, lds).
inline long resident_blocks(const void* kernel, int block, size_t lds, long fallback) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, size_t>, long> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fallback;
  const auto key = std::make_tuple(dev, kernel, block, lds);
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return fallback;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess ||
      per_cu <= 0)
    return fallback;
  const long n = (long)cus * per_cu;
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = n;
  return n;
}

}  // namespace ppo
