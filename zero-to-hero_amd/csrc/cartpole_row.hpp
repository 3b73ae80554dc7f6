// One CartPole-v1 transition for one environment, shared by the stand-alone
// environment step (cartpole.hip) and the fused rollout (mlp.hip).
//
// The dynamics are the classic cart-pole of Barto, Sutton & Anderson (1983)
// with the constants and semi-implicit conventions of gymnasium's
// CartPoleEnv (gymnasium >= 1.3, rl/uv.lock; not part of the reference
// sources): gravity 9.8, cart mass 1.0, pole mass 0.1, half-length 0.5,
// force 10.0, tau 0.02, explicit Euler; fp64 state.  Per step, with
// F = +-10 for action 1 / 0:
//   temp   = (F + m_p l thetadot^2 sin(theta)) / (m_c + m_p)
//   thacc  = (g sin(theta) - cos(theta) temp) / (l (4/3 - m_p cos^2(theta) / (m_c + m_p)))
//   xacc   = temp - m_p l thacc cos(theta) / (m_c + m_p)
//   x += tau xdot; xdot += tau xacc; theta += tau thetadot; thetadot += tau thacc
// terminated when |x| > 2.4 or |theta| > 12 degrees; reward 1 every step;
// truncated when the episode reaches max_steps (500 for CartPole-v1).  A done
// environment is reset in the same step from the caller's uniforms,
// state_i = -0.05 + 0.1 u_i.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace ppo {

struct CartpoleStep {
  bool term, done;
};

// Reset state from four U[0,1) draws.
__device__ __forceinline__ void cartpole_reset_state(double (&s)[4], const float* u) {
#pragma clang fp contract(off)
#pragma unroll
  for (int k = 0; k < 4; ++k) s[k] = -0.05 + (0.05 - -0.05) * (double)u[k];
}

// Advance s (in place) by `action`; `steps` is the episode's step count
// before the transition and after it (0 after a reset).  Each fp64 operation
// rounds on its own, in the order gymnasium evaluates it in Python floats.
__device__ __forceinline__ CartpoleStep cartpole_advance(double (&s)[4], int action, int& steps,
                                                         int max_steps, const float* reset_u) {
#pragma clang fp contract(off)
  constexpr double kGravity = 9.8;
  constexpr double kMassCart = 1.0;
  constexpr double kMassPole = 0.1;
  constexpr double kLength = 0.5;  // half the pole's length
  constexpr double kForceMag = 10.0;
  constexpr double kTau = 0.02;
  constexpr double kXThreshold = 2.4;
  const double total_mass = kMassPole + kMassCart;
  const double polemass_length = kMassPole * kLength;
  const double theta_threshold = 12.0 * 2.0 * M_PI / 360.0;
  const double x = s[0], x_dot = s[1], theta = s[2], theta_dot = s[3];
  const double force = action == 1 ? kForceMag : -kForceMag;
  const double costheta = cos(theta);
  const double sintheta = sin(theta);
  const double temp = (force + polemass_length * (theta_dot * theta_dot) * sintheta) / total_mass;
  const double thetaacc = (kGravity * sintheta - costheta * temp) /
                          (kLength * (4.0 / 3.0 - kMassPole * (costheta * costheta) / total_mass));
  const double xacc = temp - polemass_length * thetaacc * costheta / total_mass;
  s[0] = x + kTau * x_dot;
  s[1] = x_dot + kTau * xacc;
  s[2] = theta + kTau * theta_dot;
  s[3] = theta_dot + kTau * thetaacc;
  CartpoleStep r;
  r.term = s[0] < -kXThreshold || s[0] > kXThreshold || s[2] < -theta_threshold ||
           s[2] > theta_threshold;
  const int t = steps + 1;
  r.done = r.term || t >= max_steps;
  if (r.done) cartpole_reset_state(s, reset_u);
  steps = r.done ? 0 : t;
  return r;
}

}  // namespace ppo
