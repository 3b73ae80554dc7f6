// clip_grad_norm_ + Adam: the update arithmetic (update.hip's kernels) and
// the entry point the fused MLP minibatch step (mlp.hip) enqueues.  The fp32
// arithmetic follows torch's multi-tensor Adam op by op (lerp for the first
// moment, mul + addcmul for the second, sqrt / bias-correction / eps /
// addcdiv for the update), each operation rounded separately, and the clip
// coefficient follows torch's two-level _get_total_norm.
#pragma once

#include "common.hpp"

namespace ppo {

struct AdamScalars {
  // host-formed scalars (used when no device step counter is given)
  float max_norm;      // clip threshold
  float beta1_w;       // 1 - beta1, the lerp weight
  float beta2;
  float one_m_beta2;   // 1 - beta2
  float bc2_sqrt;      // sqrt(1 - beta2^step)
  float eps;
  float neg_step;      // -(lr / (1 - beta1^step))
  int clip;            // 0: no clipping (max_norm <= 0)
  // for the device step counter: the Python doubles the bias corrections
  // are formed from
  double lr_d, beta1_d, beta2_d;
};

// Host-side scalars exactly as torch forms them: Python doubles, rounded to
// fp32 where the tensor op consumes them.  Defined in update.hip.
AdamScalars make_adam_scalars(const ppo_adam_params* hp);

// Bias-correction scalars for `step`, formed as torch forms them in Python
// doubles (1 - beta^t, lr / bc1 * -1, bc2 ** 0.5) and rounded to fp32.
__device__ inline void adam_step_scalars_at(AdamScalars& s, double step) {
  const double bc1 = 1.0 - pow(s.beta1_d, step);
  const double bc2 = 1.0 - pow(s.beta2_d, step);
  s.neg_step = (float)((s.lr_d / bc1) * -1.0);
  s.bc2_sqrt = (float)sqrt(bc2);
}

// One element: gradient g (clipped by coef when clipping), moments m, v and
// parameter p in; the clipped gradient, the new moments and the new
// parameter out.
// The arithmetic is spelled out, FMAs included, so that every kernel that
// inlines it rounds the same way (HIP's __f*_rn helpers are plain operators
// that the backend may fuse differently in different inlined copies): the
// fused forms are those of torch's elementwise kernels (lerp_, addcmul_ and
// addcdiv_ each evaluate as one FMA); everything else is rounded on its
// own, the clipped gradient included (clip_grad_norm_ stores it before Adam
// reads it); sqrt and divides are correctly rounded.
__device__ __forceinline__ void adam_elem(const AdamScalars& s, float coef, float g, float m,
                                          float v, float p, float& go, float& mo, float& vo,
                                          float& po) {
#pragma clang fp contract(off)
  go = s.clip ? g * coef : g;
  // exp_avg.lerp_(grad, 1 - beta1), weight < 0.5: m + w * (g - m)
  mo = fmaf(s.beta1_w, go - m, m);
  // exp_avg_sq.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
  vo = fmaf(s.one_m_beta2 * go, go, v * s.beta2);
  // denom = sqrt(v) / sqrt(1 - beta2^t) + eps;  p.addcdiv_(m, denom, value=-lr / (1 - beta1^t))
  const float denom = sqrtf(vo) / s.bc2_sqrt + s.eps;
  po = fmaf(s.neg_step, mo / denom, p);
}

// The total norm and clip coefficient from the per-tensor norms (fp32, in
// tensor order: torch's _get_total_norm), rounded op by op.
__device__ inline float adam_coef_from_norms(const AdamScalars& s, const float* norms, int nt,
                                             float& norm) {
#pragma clang fp contract(off)
  float total_sq = 0.0f;
  for (int q = 0; q < nt; ++q) total_sq = total_sq + norms[q] * norms[q];
  norm = sqrtf(total_sq);
  float coef = 1.0f;
  if (s.clip) {
    const float c = s.max_norm / (norm + 1e-6f);
    coef = c < 1.0f ? c : 1.0f;
  }
  return coef;
}

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
