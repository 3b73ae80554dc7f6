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

// Workspace header.  Cross-workgroup results are always combined by a
// separate one-block kernel launched after the producer on the same stream:
// on gfx950 an in-kernel "last block finalises" handshake needs an agent-scope
// release fence per workgroup, which compiles to a full L2 write-back
// (buffer_wbl2) and costs far more than one extra launch.
struct WsHeader {
  float stats[4];         // {mean, std, denom, 0} written by the stats finaliser
};
static_assert(sizeof(WsHeader) <= kHeaderBytes, "header too big");

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline int hip_status(hipError_t e) { return e == hipSuccess ? PPO_OK : PPO_ERR_HIP_BASE + (int)e; }

// Launch-error check after a hipLaunchKernelGGL.
inline int last_launch_status() { return hip_status(hipGetLastError()); }

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// Block-wide sum of K doubles per thread; result valid in thread 0.
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
  if (threadIdx.x == 0) {
    const int nw = blockDim.x / kWave;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      double s = 0.0;
      for (int w = 0; w < nw; ++w) s += s_part[w][k];
      x[k] = s;
    }
  }
  __syncthreads();
}

// Sums of `count` partial (n, sum x, sum x^2, pad) quadruples, combined by
// one block in a fixed order (contiguous range per thread, then the block
// tree), so every block that calls this gets bit-identical totals.  Result
// valid in thread 0.
__device__ inline void sum_partials(const double* part, long count, double (&tot)[3]) {
  tot[0] = tot[1] = tot[2] = 0.0;
  const long per = (count + blockDim.x - 1) / blockDim.x;
  const long lo = (long)threadIdx.x * per;
  const long hi = lo + per < count ? lo + per : count;
  for (long i = lo; i < hi; ++i) {
    tot[0] += part[4 * i + 0];
    tot[1] += part[4 * i + 1];
    tot[2] += part[4 * i + 2];
  }
  block_sum<3>(tot);
}

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
