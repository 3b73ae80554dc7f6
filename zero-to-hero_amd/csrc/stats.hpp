// Advantage-normalisation statistics shared by the fused GAE+normalise path
// and the stand-alone normaliser (rl/deep/agents/ppo.py:126-127).
#pragma once

#include "common.hpp"

namespace ppo {

// One-block kernel body, run after every producer block has stored its
// (n, mean, M2) partial (a previous launch on the same stream).  Computes mean and the unbiased std in fp64, rounds both to fp32
// (torch returns fp32 0-d tensors for .mean() / .std()), and forms the fp32
// denominator std + eps exactly as `advantages.std() + 1e-8` does.  For n <= 1
// the normaliser must be the identity (the reference skips it when
// len(advantages) <= 1), so mean = 0 and denom = 1 are stored instead.
__device__ inline void finalize_stats(const double* partials, long count, double eps,
                                      WsHeader* hdr, float* stats_out) {
  Moments m = combine_partials(partials, count);
  if (threadIdx.x == 0) {
    float mean_f, std_f, denom;
    if (m.n > 1.0) {
      const double var = m.m2 / (m.n - 1.0);
      mean_f = (float)m.mean;
      std_f = (float)sqrt(var);
      denom = std_f + (float)eps;
      hdr->stats[0] = mean_f;
      hdr->stats[2] = denom;
    } else {
      mean_f = (float)m.mean;
      std_f = __builtin_nanf("");
      hdr->stats[0] = 0.0f;
      hdr->stats[2] = 1.0f;
    }
    hdr->stats[1] = std_f;
    if (stats_out) {
      stats_out[0] = mean_f;
      stats_out[1] = std_f;
    }
  }
}

// Enqueue the one-block finaliser over `count` partials.  Defined in
// adv_norm.hip.
int launch_finalize_stats(const double* partials, long count, double eps, WsHeader* hdr,
                          float* stats_out, hipStream_t stream);

// Enqueue out[i] = (adv[i] - mean) / denom (fp32) where mean/denom are the
// values finalize_stats() stored in `hdr` earlier on the same stream.
// Defined in adv_norm.hip.
int launch_normalize(const float* adv, float* out, long n, const WsHeader* hdr,
                     hipStream_t stream);

}  // namespace ppo
