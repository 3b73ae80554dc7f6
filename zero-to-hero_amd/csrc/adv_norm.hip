// Advantage normalisation (rl/deep/agents/ppo.py:126-127):
//     if len(advantages) > 1:
//         advantages = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
// Three kernels: a moments pass (fp64 Chan combine per thread, then per
// block), a one-block finaliser combining the block partials in a fixed order,
// and an fp32 elementwise pass.
#include <algorithm>

#include "common.hpp"
#include "stats.hpp"

namespace ppo {
namespace {

constexpr long kMaxStatBlocks = 2048;

long stat_blocks(long n) {
  const long groups = (n + 3) / 4;
  long b = (groups + kBlock - 1) / kBlock;
  return std::max(1L, std::min(b, kMaxStatBlocks));
}

// Moments of 4 values as one (n, mean, M2) triple.
__device__ __forceinline__ Moments moments4(float x0, float x1, float x2, float x3) {
  const double a = x0, b = x1, c = x2, d = x3;
  const double mean = (a + b + c + d) * 0.25;
  const double da = a - mean, db = b - mean, dc = c - mean, dd = d - mean;
  return {4.0, mean, da * da + db * db + dc * dc + dd * dd};
}

template <bool kVec>
__global__ void __launch_bounds__(kBlock) adv_moments_kernel(const float* adv, long n,
                                                             double* partial) {
  Moments m = {0.0, 0.0, 0.0};
  const long stride = (long)gridDim.x * blockDim.x;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long tail_start = 0;
  if constexpr (kVec) {
    const long n4 = n / 4;
    const float4* a4 = reinterpret_cast<const float4*>(adv);
    for (long i = gid; i < n4; i += stride) {
      const float4 x = a4[i];
      m = moments_combine(m, moments4(x.x, x.y, x.z, x.w));
    }
    tail_start = n4 * 4;
  }
  for (long i = tail_start + gid; i < n; i += stride) {
    const Moments one = {1.0, (double)adv[i], 0.0};
    m = moments_combine(m, one);
  }
  m = block_moments(m);
  if (threadIdx.x == 0) {
    partial[blockIdx.x * 4 + 0] = m.n;
    partial[blockIdx.x * 4 + 1] = m.mean;
    partial[blockIdx.x * 4 + 2] = m.m2;
    partial[blockIdx.x * 4 + 3] = 0.0;
  }
}

__global__ void __launch_bounds__(kBlock) finalize_stats_kernel(const double* partial, long count,
                                                                double eps, WsHeader* hdr,
                                                                float* stats_out) {
  finalize_stats(partial, count, eps, hdr, stats_out);
}

template <bool kVec>
__global__ void __launch_bounds__(kBlock) normalize_kernel(const float* adv, float* out, long n,
                                                           const WsHeader* hdr) {
  const float mean = hdr->stats[0];
  const float denom = hdr->stats[2];
  const long stride = (long)gridDim.x * blockDim.x;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long tail_start = 0;
  if constexpr (kVec) {
    const long n4 = n / 4;
    const float4* a4 = reinterpret_cast<const float4*>(adv);
    float4* o4 = reinterpret_cast<float4*>(out);
    for (long i = gid; i < n4; i += stride) {
      const float4 x = a4[i];
      float4 y;
      y.x = (x.x - mean) / denom;
      y.y = (x.y - mean) / denom;
      y.z = (x.z - mean) / denom;
      y.w = (x.w - mean) / denom;
      o4[i] = y;
    }
    tail_start = n4 * 4;
  }
  for (long i = tail_start + gid; i < n; i += stride) out[i] = (adv[i] - mean) / denom;
}

}  // namespace

int launch_finalize_stats(const double* partials, long count, double eps, WsHeader* hdr,
                          float* stats_out, hipStream_t stream) {
  hipLaunchKernelGGL(finalize_stats_kernel, dim3(1), dim3(kBlock), 0, stream, partials, count,
                     eps, hdr, stats_out);
  return last_launch_status();
}

int launch_normalize(const float* adv, float* out, long n, const WsHeader* hdr,
                     hipStream_t stream) {
  if (n <= 0) return PPO_OK;
  const bool vec = aligned(adv, 16) && aligned(out, 16);
  const long work = vec ? (n + 3) / 4 : n;
  long blocks = (work + kBlock - 1) / kBlock;
  blocks = std::max(1L, std::min(blocks, 8192L));
  if (vec)
    hipLaunchKernelGGL(normalize_kernel<true>, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       adv, out, n, hdr);
  else
    hipLaunchKernelGGL(normalize_kernel<false>, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       adv, out, n, hdr);
  return last_launch_status();
}

}  // namespace ppo

extern "C" size_t ppo_adv_norm_workspace_bytes(int64_t n) {
  using namespace ppo;
  if (n <= 0) return kHeaderBytes;
  return kHeaderBytes + align_up((size_t)stat_blocks(n) * 4 * sizeof(double), 256);
}

extern "C" int ppo_adv_norm_f32(const float* adv, int64_t n, double eps, float* out,
                                float* stats_out, void* workspace, size_t workspace_bytes,
                                void* stream_ptr) {
  using namespace ppo;
  if (n < 0) return PPO_ERR_INVALID_ARG;
  if (n == 0) return PPO_OK;
  if (!adv || !out) return PPO_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < ppo_adv_norm_workspace_bytes(n)) return PPO_ERR_WORKSPACE;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  WsHeader* hdr = reinterpret_cast<WsHeader*>(workspace);
  double* partial = reinterpret_cast<double*>(static_cast<char*>(workspace) + kHeaderBytes);
  const long blocks = stat_blocks(n);
  if (aligned(adv, 16))
    hipLaunchKernelGGL(adv_moments_kernel<true>, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       adv, (long)n, partial);
  else
    hipLaunchKernelGGL(adv_moments_kernel<false>, dim3((unsigned)blocks), dim3(kBlock), 0,
                       stream, adv, (long)n, partial);
  int st = last_launch_status();
  if (st) return st;
  if ((st = launch_finalize_stats(partial, blocks, eps, hdr, stats_out, stream))) return st;
  return launch_normalize(adv, out, n, hdr, stream);
}
