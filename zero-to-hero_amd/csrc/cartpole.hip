// Vectorised CartPole-v1 on the device: the environment the reference trains
// on (rl/deep/cli.py:179-180 gym.make("CartPole-v1"), stepped one transition
// at a time by rl/deep/runner.py:56-74), for N environments per launch.
//
// The dynamics are the classic cart-pole of Barto, Sutton & Anderson (1983)
// with the constants and semi-implicit conventions of gymnasium's
// CartPoleEnv (gymnasium >= 1.3, rl/uv.lock; not part of the reference
// sources): gravity 9.8, cart mass 1.0, pole mass 0.1, half-length 0.5,
// force 10.0, tau 0.02, explicit Euler; fp64 state, observations rounded to
// fp32.  Per step, with F = +-10 for action 1 / 0:
//   temp   = (F + m_p l thetadot^2 sin(theta)) / (m_c + m_p)
//   thacc  = (g sin(theta) - cos(theta) temp) / (l (4/3 - m_p cos^2(theta) / (m_c + m_p)))
//   xacc   = temp - m_p l thacc cos(theta) / (m_c + m_p)
//   x += tau xdot; xdot += tau xacc; theta += tau thetadot; thetadot += tau thacc
// terminated when |x| > 2.4 or |theta| > 12 degrees; reward 1 every step;
// truncated when the episode reaches max_steps (500 for CartPole-v1).  A done
// environment is reset in the same step from the caller's uniforms,
// state_i = -0.05 + 0.1 u_i, and its reset observation is returned (the
// terminal observation is not needed: the reference bootstraps nothing at an
// episode end, ppo.py:179).
#include <math.h>

#include "common.hpp"

// Each fp64 operation rounds on its own, as the Python-float restatement
// does: no contraction into fused multiply-adds in this file.
#pragma clang fp contract(off)

namespace ppo {
namespace {

constexpr double kGravity = 9.8;
constexpr double kMassCart = 1.0;
constexpr double kMassPole = 0.1;
constexpr double kLength = 0.5;  // half the pole's length
constexpr double kForceMag = 10.0;
constexpr double kTau = 0.02;
constexpr double kXThreshold = 2.4;

__device__ __forceinline__ void reset_state(double (&s)[4], const float* u) {
#pragma unroll
  for (int k = 0; k < 4; ++k) s[k] = -0.05 + (0.05 - -0.05) * (double)u[k];
}

__global__ void __launch_bounds__(kBlock) cartpole_step_kernel(
    double* __restrict__ state, int32_t* __restrict__ steps, const int32_t* __restrict__ actions,
    const float* __restrict__ uniforms, int max_steps, float* __restrict__ obs,
    float* __restrict__ rewards, uint8_t* __restrict__ dones, uint8_t* __restrict__ terminated,
    float* __restrict__ ep_return, double* __restrict__ done_sum,
    int32_t* __restrict__ done_count, long N) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  // operation order as gymnasium evaluates it in Python floats
  const double total_mass = kMassPole + kMassCart;
  const double polemass_length = kMassPole * kLength;
  const double theta_threshold = 12.0 * 2.0 * M_PI / 360.0;
  double s[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) s[k] = state[n * 4 + k];
  const double x = s[0], x_dot = s[1], theta = s[2], theta_dot = s[3];
  const double force = actions[n] == 1 ? kForceMag : -kForceMag;
  const double costheta = cos(theta);
  const double sintheta = sin(theta);
  const double temp = (force + polemass_length * (theta_dot * theta_dot) * sintheta) / total_mass;
  const double thetaacc = (kGravity * sintheta - costheta * temp) /
                          (kLength * (4.0 / 3.0 - kMassPole * (costheta * costheta) / total_mass));
  const double xacc = temp - polemass_length * thetaacc * costheta / total_mass;
  const double nx = x + kTau * x_dot;
  const double nx_dot = x_dot + kTau * xacc;
  const double ntheta = theta + kTau * theta_dot;
  const double ntheta_dot = theta_dot + kTau * thetaacc;
  const bool term = nx < -kXThreshold || nx > kXThreshold || ntheta < -theta_threshold ||
                    ntheta > theta_threshold;
  const int t = steps[n] + 1;
  const bool trunc = t >= max_steps;
  const bool done = term || trunc;
  double o[4] = {nx, nx_dot, ntheta, ntheta_dot};
  if (done) reset_state(o, uniforms + n * 4);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    state[n * 4 + k] = o[k];
    obs[n * 4 + k] = (float)o[k];
  }
  steps[n] = done ? 0 : t;
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
  reset_state(o, uniforms + n * 4);
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
