// The update half of ppo_adam_clip_f32 for callers that already hold the
// gradients' sums of squares (the fused MLP step, mlp.hip).
#pragma once

#include "common.hpp"

namespace ppo {

// Enqueue clip_grad_norm_ + Adam over nt tensors whose per-tensor sums of
// squared gradients are partials[part_start[k] .. part_start[k + 1]) (fp64,
// summed in that order), written by an earlier launch on the same stream.
// With hp->step_counter the earlier launch must also have incremented the
// counter.  Defined in update.hip.
int launch_adam_presummed(int nt, float* const* params, float* const* grads,
                          float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                          const ppo_adam_params* hp, const double* partials,
                          const long* part_start, float* grad_norm_out, hipStream_t stream);

}  // namespace ppo
