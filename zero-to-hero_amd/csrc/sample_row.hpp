// Categorical action selection for one row (rl/deep/agents/ppo.py:65-79,
// select_action), shared by the sampling kernels (sample.hip) and the fused
// MLP forward + sampling kernel (mlp.hip).
//
// The draw is the inverse CDF at the caller's uniform u: with m = max_j z_j,
// e_j = exp(z_j - m), s = sum_j e_j, the action is the first j whose running
// sum of e exceeds u*s (the last reachable action if rounding leaves u*s at
// or above the total), and its log-probability is (z_a - m) - log s (the
// log_softmax that Categorical.__init__ applies, ppo.py:70-71).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace ppo {

__device__ __forceinline__ void sample_cat_row(const float* zr, int A, float u, int& action,
                                               float& logp) {
  float m = -INFINITY;
  for (int j = 0; j < A; ++j) m = fmaxf(m, zr[j]);
  float s = 0.0f;
  for (int j = 0; j < A; ++j) s += expf(zr[j] - m);
  const float target = u * s;
  float c = 0.0f;
  int a = -1, last_pos = 0;
  for (int j = 0; j < A; ++j) {
    const float e = expf(zr[j] - m);
    c += e;
    if (e > 0.0f) last_pos = j;
    if (a < 0 && target < c) a = j;
  }
  if (a < 0) a = last_pos;
  action = a;
  logp = (zr[a] - m) - logf(s);
}

}  // namespace ppo
