// Vectorised CartPole-v1 on the device: the environment the reference trains
// on (rl/deep/cli.py:179-180 gym.make("CartPole-v1"), stepped one transition
// at a time by rl/deep/runner.py:56-74), for N environments per launch.  The
// transition itself (gymnasium's CartPoleEnv dynamics, fp64) is
// cartpole_row.hpp; here one thread steps one environment, writes its fp32
// observation, reward and done flag, and keeps its episode tally.  A done
// environment's reset observation is returned (the terminal observation is
// not needed: the reference bootstraps nothing at an episode end,
// ppo.py:179).
#include <math.h>

#include "cartpole_row.hpp"
#include "common.hpp"

// Each fp64 operation rounds on its own, as the Python-float restatement
// does: no contraction into fused multiply-adds in this file.
#pragma clang fp contract(off)

namespace ppo {
namespace {

__global__ void __launch_bounds__(kBlock) cartpole_step_kernel(
    double* __restrict__ state, int32_t* __restrict__ steps, const int32_t* __restrict__ actions,
    const float* __restrict__ uniforms, int max_steps, float* __restrict__ obs,
    float* __restrict__ rewards, uint8_t* __restrict__ dones, uint8_t* __restrict__ terminated,
    float* __restrict__ ep_return, double* __restrict__ done_sum,
    int32_t* __restrict__ done_count, long N) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  double s[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) s[k] = state[n * 4 + k];
  int t = steps[n];
  const CartpoleStep r = cartpole_advance(s, actions[n], t, max_steps, uniforms + n * 4);
  const bool term = r.term, done = r.done;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    state[n * 4 + k] = s[k];
    obs[n * 4 + k] = (float)s[k];
  }
  steps[n] = t;
  rewards[n] = 1.0f;
  dones[n] = done ? 1 : 0;
  if (terminated) terminated[n] = term ? 1 : 0;
  if (ep_return) {
    const float ret = ep_return[n] + 1.0f;
    if (done) {
      done_sum[n] += (double)ret;
      done_count[n] += 1;
    }
    ep_return[n] = done ? 0.0f : ret;
  }
}

__global__ void __launch_bounds__(kBlock) cartpole_reset_kernel(double* __restrict__ state,
                                                                int32_t* __restrict__ steps,
                                                                const float* __restrict__ uniforms,
                                                                float* __restrict__ obs, long N) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  double o[4];
  cartpole_reset_state(o, uniforms + n * 4);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    state[n * 4 + k] = o[k];
    obs[n * 4 + k] = (float)o[k];
  }
  steps[n] = 0;
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_cartpole_reset(double* state, int32_t* steps, const float* uniforms,
                                  float* obs_out, int64_t N, void* stream) {
  using namespace ppo;
  if (N < 0) return PPO_ERR_INVALID_ARG;
  if (N == 0) return PPO_OK;
  if (!state || !steps || !uniforms || !obs_out) return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31)) return PPO_ERR_TOO_LARGE;
  hipLaunchKernelGGL(cartpole_reset_kernel, dim3((unsigned)((N + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream), state, steps,
                     uniforms, obs_out, (long)N);
  return last_launch_status();
}

extern "C" int ppo_cartpole_step(double* state, int32_t* steps, const int32_t* actions,
                                 const float* reset_uniforms, int32_t max_steps, float* obs_out,
                                 float* rewards_out, uint8_t* dones_out,
                                 uint8_t* terminated_out, float* episode_return,
                                 double* completed_sum, int32_t* completed_count, int64_t N,
                                 void* stream) {
  using namespace ppo;
  if (N < 0 || max_steps < 1) return PPO_ERR_INVALID_ARG;
  if ((episode_return == nullptr) != (completed_sum == nullptr) ||
      (episode_return == nullptr) != (completed_count == nullptr))
    return PPO_ERR_INVALID_ARG;
  if (N == 0) return PPO_OK;
  if (!state || !steps || !actions || !reset_uniforms || !obs_out || !rewards_out || !dones_out)
    return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31)) return PPO_ERR_TOO_LARGE;
  hipLaunchKernelGGL(cartpole_step_kernel, dim3((unsigned)((N + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, reinterpret_cast<hipStream_t>(stream), state, steps,
                     actions, reset_uniforms, (int)max_steps, obs_out, rewards_out, dones_out,
                     terminated_out, episode_return, completed_sum, completed_count, (long)N);
  return last_launch_status();
}
