/*
 * CPU restatement of the reference GAE (test infrastructure only: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the
 * checker; the product path never calls it).
 *
 * Follows rl/deep/agents/ppo.py:173-193 (PPOAgent._advantages) and :124
 * (returns = advantages + old_values), generalised to N envs stored [T,N]
 * env-contiguous with a bootstrap last_value[N] (NULL = zeros, the reference's
 * `next_value = 0.0` at :176).  Arithmetic is IEEE binary64 in the exact
 * order Python evaluates the reference's expressions, left to right:
 *     mask  = 1.0 - float(done)                               (:179)
 *     delta = (reward + (gamma*next_value)*mask) - value      (:180-184)
 *     adv   = delta + ((gamma*lam)*mask)*adv                  (:185-188)
 *     next_value = value                                      (:190)
 * followed by the fp32 cast of torch.as_tensor(..., float32) (:193).
 * Build with -ffp-contract=off so no step is fused into an FMA.
 */
#include <stddef.h>
#include <stdint.h>

void gae_ref_f64(const float* rewards, const float* values, const uint8_t* dones,
                 const float* last_value, int64_t T, int64_t N, double gamma,
                 double lam, float* adv_out, float* ret_out) {
  const double gl = gamma * lam; /* Python: gamma * gae_lambda, rounded once */
  for (int64_t n = 0; n < N; ++n) {
    double advantage = 0.0;
    double next_value = last_value ? (double)last_value[n] : 0.0;
    for (int64_t t = T - 1; t >= 0; --t) {
      const int64_t i = t * N + n;
      const double mask = 1.0 - (dones[i] ? 1.0 : 0.0);
      const double value = (double)values[i];
      const double delta = ((double)rewards[i] + (gamma * next_value) * mask) - value;
      advantage = delta + (gl * mask) * advantage;
      adv_out[i] = (float)advantage;
      if (ret_out) ret_out[i] = (float)advantage + values[i]; /* fp32 add */
      next_value = value;
    }
  }
}
