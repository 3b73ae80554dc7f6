// Batched action selection (rl/deep/agents/ppo.py:65-79, select_action) for
// N environments per launch, written straight into a rollout buffer row.
//
// Categorical: Categorical(logits).sample() draws from softmax(logits); here
// the draw is the inverse CDF at the caller's uniform u, so that a rollout is
// a deterministic function of (logits, u): with m = max_j z_j,
// e_j = exp(z_j - m), s = sum_j e_j, the action is the first j whose running
// sum of e exceeds u*s, and its log-probability is (z_a - m) - log s (the
// log_softmax that Categorical.__init__ applies, ppo.py:70-71).
// Gaussian: Normal(mu, sigma).sample() is mu + sigma*eps with the caller's eps.
//
// These launches are latency-bound (N rows of a few floats per env step):
// one thread per row for A <= kRowMaxA, one wave per row above that.
#include <algorithm>

#include "common.hpp"
#include "sample_row.hpp"

namespace ppo {
namespace {

constexpr int kRowMaxA = 64;
constexpr int kMaxSampleDim = 24;

__global__ void __launch_bounds__(kBlock) sample_cat_row_kernel(const float* __restrict__ z,
                                                                long N, int A,
                                                                const float* __restrict__ u,
                                                                int32_t* act, float* logp,
                                                                const float* val, float* val_out) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  int a;
  float lp;
  sample_cat_row(z + n * A, A, u[n], a, lp);
  act[n] = a;
  logp[n] = lp;
  if (val && val_out) val_out[n] = val[n];
}

// One wave per row: lane l owns the contiguous chunk [l*c, (l+1)*c) of the row,
// so lane order is index order and a wave prefix sum of the lane totals
// locates the chunk holding the sample.
__global__ void __launch_bounds__(kBlock) sample_cat_wave_kernel(const float* __restrict__ z,
                                                                 long N, int A,
                                                                 const float* __restrict__ u,
                                                                 int32_t* act, float* logp,
                                                                 const float* val,
                                                                 float* val_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const long n = ((long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (n >= N) return;  // whole waves leave together
  const float* zr = z + n * A;
  const int c = (A + kWave - 1) / kWave;
  const int lo = std::min(A, lane * c), hi = std::min(A, lo + c);
  float m = -INFINITY;
  for (int j = lo; j < hi; ++j) m = fmaxf(m, zr[j]);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  float part = 0.0f;
  int last_pos = -1;
  for (int j = lo; j < hi; ++j) {
    const float e = expf(zr[j] - m);
    part += e;
    if (e > 0.0f) last_pos = j;
  }
  // inclusive prefix over lanes (lane order = index order)
  float incl = part;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  const float s = __shfl(incl, kWave - 1, kWave);
  const float target = u[n] * s;
  // first lane whose inclusive total exceeds the target
  const unsigned long long hit = __ballot(target < incl);
  int a;
  if (hit) {
    const int l = __ffsll((long long)hit) - 1;
    const float before = __shfl(incl - part, l, kWave);
    a = -1;
    if (lane == l) {
      float cc = before;
      for (int j = lo; j < hi; ++j) {
        cc += expf(zr[j] - m);
        if (target < cc) { a = j; break; }
      }
      if (a < 0) a = last_pos >= 0 ? last_pos : lo;
    }
    a = __shfl(a, l, kWave);
  } else {
    int lp = last_pos;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) lp = max(lp, __shfl_xor(lp, off, kWave));
    a = lp >= 0 ? lp : 0;
  }
  if (lane == 0) {
    act[n] = a;
    logp[n] = (zr[a] - m) - logf(s);
    if (val && val_out) val_out[n] = val[n];
  }
}

__global__ void __launch_bounds__(kBlock) sample_gauss_kernel(const float* __restrict__ mu,
                                                              const float* __restrict__ log_std,
                                                              long N, int D,
                                                              const float* __restrict__ eps,
                                                              float* act, float* logp,
                                                              const float* val, float* val_out) {
  __shared__ float s_scale[kMaxSampleDim], s_inv2var[kMaxSampleDim], s_logscale[kMaxSampleDim];
  if (threadIdx.x < D) {
    const float scale = expf(log_std[threadIdx.x]);
    s_scale[threadIdx.x] = scale;
    s_inv2var[threadIdx.x] = 1.0f / (2.0f * (scale * scale));
    s_logscale[threadIdx.x] = logf(scale);
  }
  __syncthreads();
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float kLogSqrt2Pi = 0.91893853320467274178f;  // log(sqrt(2*pi))
  float lp = 0.0f;
  for (int d = 0; d < D; ++d) {
    const float m = mu[n * D + d];
    const float x = m + s_scale[d] * eps[n * D + d];
    act[n * D + d] = x;
    const float diff = x - m;
    lp += ((-(diff * diff)) * s_inv2var[d] - s_logscale[d]) - kLogSqrt2Pi;
  }
  logp[n] = lp;
  if (val && val_out) val_out[n] = val[n];
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_sample_cat_f32(const float* logits, int64_t N, int32_t A, const float* uniforms,
                                  int32_t* actions_out, float* logp_out, const float* values,
                                  float* values_out, void* stream_ptr) {
  using namespace ppo;
  if (N < 0 || A <= 0) return PPO_ERR_INVALID_ARG;
  if (N == 0) return PPO_OK;
  if (!logits || !uniforms || !actions_out || !logp_out) return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31) || (long)N * A > (1L << 50)) return PPO_ERR_TOO_LARGE;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (A <= kRowMaxA) {
    const long blocks = (N + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(sample_cat_row_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       logits, (long)N, (int)A, uniforms, actions_out, logp_out, values,
                       values_out);
  } else {
    const long blocks = (N * kWave + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(sample_cat_wave_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       logits, (long)N, (int)A, uniforms, actions_out, logp_out, values,
                       values_out);
  }
  return last_launch_status();
}

extern "C" int ppo_sample_gauss_f32(const float* mu, const float* log_std, int64_t N, int32_t D,
                                    const float* normals, float* actions_out, float* logp_out,
                                    const float* values, float* values_out, void* stream_ptr) {
  using namespace ppo;
  if (N < 0 || D <= 0) return PPO_ERR_INVALID_ARG;
  if (D > kMaxSampleDim) return PPO_ERR_TOO_LARGE;
  if (N == 0) return PPO_OK;
  if (!mu || !log_std || !normals || !actions_out || !logp_out) return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31)) return PPO_ERR_TOO_LARGE;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const long blocks = (N + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(sample_gauss_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream, mu,
                     log_std, (long)N, (int)D, normals, actions_out, logp_out, values,
                     values_out);
  return last_launch_status();
}
