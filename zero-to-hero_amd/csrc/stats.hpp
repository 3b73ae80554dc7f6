// Advantage-normalisation statistics shared by the fused GAE+normalise path
// and the stand-alone normaliser (rl/deep/agents/ppo.py:126-127).
#pragma once

#include "common.hpp"

namespace ppo {

// Normaliser parameters from the block partials (n, sum x, sum x^2 in fp64),
// combined in a fixed order by one block (the same order in every block that
// calls this, so every block derives bit-identical values).  mean and the
// unbiased std, var = (sum x^2 - (sum x)^2 / n) / (n - 1), are formed in fp64
// (relative error ~1e-16 * (1 + mean^2/var), i.e. exact to fp32 unless
// |mean|/std exceeds ~1e4) and rounded to fp32 (torch returns fp32 0-d tensors for .mean() /
// .std()), and the denominator is the fp32 sum std + eps exactly as
// `advantages.std() + 1e-8` forms it.  For n <= 1 the normaliser must be the
// identity (the reference skips it when len(advantages) <= 1): mean 0 and
// denominator 1 are returned instead.  Result valid in thread 0.
struct NormParams {
  float mean_used, denom;  // what the elementwise pass applies
  float mean, std;         // what is reported
};

__device__ inline NormParams norm_params(const double* partials, long count, double eps) {
  double tot[3];
  sum_partials(partials, count, tot);
  const double n = tot[0];
  const double mean = tot[1] / n;
  NormParams r;
  r.mean = (float)mean;
  if (n > 1.0) {
    const double m2 = tot[2] - tot[1] * mean;
    r.std = (float)sqrt((m2 > 0.0 ? m2 : 0.0) / (n - 1.0));
    r.mean_used = r.mean;
    r.denom = r.std + (float)eps;
  } else {
    r.std = __builtin_nanf("");
    r.mean_used = 0.0f;
    r.denom = 1.0f;
  }
  return r;
}

// Enqueue the one-block kernel that turns `count` (n, sum, sum of squares)
// partials into the normaliser parameters in hdr->stats ({mean used, std,
// denominator}) and {mean, std} in stats_out (if not null).  Defined in
// adv_norm.hip.
int launch_finalize_stats(const double* partials, long count, double eps, WsHeader* hdr,
                          float* stats_out, hipStream_t stream);

// Enqueue the normaliser: mean/denom from the `count` (n, sum, sum of
// squares) partials left in the workspace by the previous kernel on the same
// stream (also stored in hdr->stats, and {mean, std} in stats_out if not
// null), then out[i] = (adv[i] - mean) / denom in fp32 over n elements.  With
// few partials and 16-byte aligned buffers this is one kernel whose blocks
// each combine the partials; otherwise a one-block kernel precedes the
// elementwise pass.
// Defined in adv_norm.hip.
int launch_normalize(const double* partials, long count, double eps, const float* adv, float* out,
                     long n, WsHeader* hdr, float* stats_out, hipStream_t stream);

}  // namespace ppo
