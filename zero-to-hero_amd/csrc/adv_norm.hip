// Advantage normalisation (rl/deep/agents/ppo.py:126-127):
//     if len(advantages) > 1:
//         advantages = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
// A moments pass (fp64 sums of x and x^2 per thread, then per block), then
// the block partials combined in a fixed order and an fp32 elementwise pass:
// one kernel when the partials are few (every block combines them), else a
// one-block finaliser and the elementwise pass.
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

// Per-block (n, sum x, sum x^2) of the advantages, fp64 accumulation.
template <bool kVec>
__global__ void __launch_bounds__(kBlock) adv_moments_kernel(const float* adv, long n,
                                                             double* partial) {
  double acc[3] = {0.0, 0.0, 0.0};
  const long stride = (long)gridDim.x * blockDim.x;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long tail_start = 0;
  if constexpr (kVec) {
    const long n4 = n / 4;
    const float4* a4 = reinterpret_cast<const float4*>(adv);
    for (long i = gid; i < n4; i += stride) {
      const float4 x = a4[i];
      const double x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
      acc[0] += 4.0;
      acc[1] += (x0 + x1) + (x2 + x3);
      acc[2] += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
    }
    tail_start = n4 * 4;
  }
  for (long i = tail_start + gid; i < n; i += stride) {
    const double x = adv[i];
    acc[0] += 1.0;
    acc[1] += x;
    acc[2] += x * x;
  }
  block_sum<3>(acc);
  if (threadIdx.x == 0) {
    partial[blockIdx.x * 4 + 0] = acc[0];
    partial[blockIdx.x * 4 + 1] = acc[1];
    partial[blockIdx.x * 4 + 2] = acc[2];
    partial[blockIdx.x * 4 + 3] = 0.0;
  }
}

// One block: combine the partials (fixed order) and store the normaliser
// parameters in the workspace header (and {mean, std} in stats_out).
__global__ void __launch_bounds__(kFinalBlock) finalize_stats_kernel(const double* partials, long count,
                                                                double eps, WsHeader* hdr,
                                                                float* stats_out) {
  const NormParams np = norm_params(partials, count, eps);
  if (threadIdx.x == 0) {
    hdr->stats[0] = np.mean_used;
    hdr->stats[1] = np.std;
    hdr->stats[2] = np.denom;
    if (stats_out) {
      stats_out[0] = np.mean;
      stats_out[1] = np.std;
    }
  }
}

// Elementwise pass at full occupancy, one float4 per thread per iteration.
template <bool kVec>
__global__ void __launch_bounds__(kBlock) normalize_kernel(const float* adv, float* out, long n,
                                                           const WsHeader* hdr) {
  const float mean = hdr->stats[0];
  const float denom = hdr->stats[2];
  const long stride = (long)gridDim.x * blockDim.x;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long tail_start = 0;
  if constexpr (kVec) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const long n4 = n / 4;
    const f4* a4 = reinterpret_cast<const f4*>(adv);
    f4* o4 = reinterpret_cast<f4*>(out);
    for (long i = gid; i < n4; i += stride) {
      const f4 x = a4[i];
      f4 y;
      y[0] = (x[0] - mean) / denom;
      y[1] = (x[1] - mean) / denom;
      y[2] = (x[2] - mean) / denom;
      y[3] = (x[3] - mean) / denom;
      __builtin_nontemporal_store(y, o4 + i);
    }
    tail_start = n4 * 4;
  }
  for (long i = tail_start + gid; i < n; i += stride) out[i] = (adv[i] - mean) / denom;
}

// The finaliser fused into the elementwise pass, for few partials: every
// block derives the normaliser parameters itself with norm_params (same
// block size as the one-block finaliser, so the same fixed order and
// bit-identical values), after issuing its first kNormU float4 loads so that
// the partials' reduction overlaps them.  Block 0 also stores the parameters
// in the header and {mean, std} in stats_out.
#ifndef PPO_NORM_U
#define PPO_NORM_U 4
#endif
constexpr int kNormU = PPO_NORM_U;
constexpr long kFusedNormMaxPartials = 512;

__global__ void __launch_bounds__(kFinalBlock) normalize_stats_kernel(
    const float* adv, float* out, long n, const double* partials, long count, double eps,
    WsHeader* hdr, float* stats_out) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __shared__ float s_par[2];
  const long n4 = n / 4;
  const f4* a4 = reinterpret_cast<const f4*>(adv);
  f4* o4 = reinterpret_cast<f4*>(out);
  const long stride = (long)gridDim.x * kFinalBlock;
  const long gid = (long)blockIdx.x * kFinalBlock + threadIdx.x;
  f4 x[kNormU];
#pragma unroll
  for (int u = 0; u < kNormU; ++u) {
    const long i = gid + u * stride;
    x[u] = a4[i < n4 ? i : 0];  // unconditional (n >= 4): element 0 stands in past the end
  }
  const NormParams np = norm_params(partials, count, eps);
  if (threadIdx.x == 0) {
    s_par[0] = np.mean_used;
    s_par[1] = np.denom;
    if (blockIdx.x == 0) {
      hdr->stats[0] = np.mean_used;
      hdr->stats[1] = np.std;
      hdr->stats[2] = np.denom;
      if (stats_out) {
        stats_out[0] = np.mean;
        stats_out[1] = np.std;
      }
    }
  }
  __syncthreads();
  const float mean = s_par[0], denom = s_par[1];
#pragma unroll
  for (int u = 0; u < kNormU; ++u) {
    const long i = gid + u * stride;
    if (i < n4) {
      f4 y;
      y[0] = (x[u][0] - mean) / denom;
      y[1] = (x[u][1] - mean) / denom;
      y[2] = (x[u][2] - mean) / denom;
      y[3] = (x[u][3] - mean) / denom;
      __builtin_nontemporal_store(y, o4 + i);
    }
  }
  for (long i = gid + kNormU * stride; i < n4; i += stride) {
    const f4 v = a4[i];
    f4 y;
    y[0] = (v[0] - mean) / denom;
    y[1] = (v[1] - mean) / denom;
    y[2] = (v[2] - mean) / denom;
    y[3] = (v[3] - mean) / denom;
    __builtin_nontemporal_store(y, o4 + i);
  }
  for (long i = n4 * 4 + gid; i < n; i += stride) out[i] = (adv[i] - mean) / denom;
}

}  // namespace

int launch_finalize_stats(const double* partials, long count, double eps, WsHeader* hdr,
                          float* stats_out, hipStream_t stream) {
  hipLaunchKernelGGL(finalize_stats_kernel, dim3(1), dim3(kFinalBlock), 0, stream, partials, count, eps,
                     hdr, stats_out);
  return last_launch_status();
}

int launch_normalize(const double* partials, long count, double eps, const float* adv, float* out,
                     long n, WsHeader* hdr, float* stats_out, hipStream_t stream) {
  if (n <= 0) return PPO_OK;
  if (count <= kFusedNormMaxPartials && n >= 4 && aligned(adv, 16) && aligned(out, 16)) {
    const long per_block = (long)kFinalBlock * kNormU;
    long blocks = ((n + 3) / 4 + per_block - 1) / per_block;
    blocks = std::max(1L, std::min(blocks, 4096L));
    hipLaunchKernelGGL(normalize_stats_kernel, dim3((unsigned)blocks), dim3(kFinalBlock), 0,
                       stream, adv, out, n, partials, count, eps, hdr, stats_out);
    return last_launch_status();
  }
  int st = launch_finalize_stats(partials, count, eps, hdr, stats_out, stream);
  if (st) return st;
  const bool vec = aligned(adv, 16) && aligned(out, 16);
  const long work = vec ? (n + 3) / 4 : n;
  long blocks = (work + kBlock - 1) / kBlock;
  blocks = std::max(1L, std::min(blocks, 8192L));
  if (vec)
    hipLaunchKernelGGL(normalize_kernel<true>, dim3((unsigned)blocks), dim3(kBlock), 0, stream, adv,
                       out, n, hdr);
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
  return launch_normalize(partial, blocks, eps, adv, out, n, hdr, stats_out, stream);
}
