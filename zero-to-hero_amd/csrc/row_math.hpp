// Per-row PPO loss arithmetic shared by the fused loss kernels (loss.hip) and
// the fused MLP minibatch kernel (mlp.hip).
//
// Reference: PPOAgent._update_batch, rl/deep/agents/ppo.py:154-167:
//     ratio   = exp(lp - old_log_probs)                            (:154)
//     clipped = ratio.clamp(1 - clip, 1 + clip)                    (:155-158)
//     policy  = -minimum(ratio * adv, clipped * adv)               (:159)
//     value   = mse_loss(values, returns)                          (:160)
// and their gradients under torch autograd's rules: minimum/maximum split the
// gradient 1/2-1/2 on ties, clamp passes it at its inclusive bounds.  With
// value clipping (no reference code) the value term is
//     max((v - R)^2, (v_old + clamp(v - v_old, -c, c) - R)^2).
#pragma once

#include <hip/hip_runtime.h>
#include <float.h>
#include <math.h>

#include "ppo_amd.h"

namespace ppo {

__device__ __forceinline__ float nan_min(float u, float w) {
  if (u != u) return u;
  if (w != w) return w;
  return u < w ? u : w;
}
__device__ __forceinline__ float nan_max(float u, float w) {
  if (u != u) return u;
  if (w != w) return w;
  return u > w ? u : w;
}
// torch.clamp(x, lo, hi): NaN stays NaN.
__device__ __forceinline__ float clampf(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// Loss hyperparameters as the kernels use them (fp32, as torch's scalar
// arithmetic on fp32 tensors rounds them).
struct RowParams {
  float lo, hi, clip;  // ratio clamp bounds and the clip parameter
  float vclip;
  int use_vclip;
  float vc, ec;        // value / entropy coefficients
  float inv_b;         // 1 / minibatch rows (the means)
};

// torch: ratio.clamp(1.0 - clip, 1.0 + clip) takes Python-double bounds and
// compares in fp32.  Value clipping is on for 0 < vf_clip < inf.
inline RowParams make_row_params(const ppo_loss_params* p, long B) {
  RowParams r;
  r.lo = (float)(1.0 - p->clip_ratio);
  r.hi = (float)(1.0 + p->clip_ratio);
  r.clip = (float)p->clip_ratio;
  r.use_vclip = (p->vf_clip > 0.0 && p->vf_clip < INFINITY) ? 1 : 0;
  r.vclip = (float)p->vf_clip;
  r.vc = (float)p->value_coef;
  r.ec = (float)p->entropy_coef;
  r.inv_b = 1.0f / (float)B;
  return r;
}

// Per-row inputs other than the logits/mu.
struct RowIn {
  float old_lp, adv, ret, v, vo;
};

struct RowOut {
  float g_lp;     // dloss/dlog_prob for this row
  float dval;     // dloss/dvalue for this row
  float pol, vl, kl, clipped;
};

// Everything per row that does not depend on the policy family: ratio,
// clipped surrogate, value loss, their gradients.  `P` carries the fields of
// RowParams.
template <typename P>
__device__ __forceinline__ RowOut ppo_row_math(const P& a, const RowIn& in, float lp) {
  RowOut o;
  const float A = in.adv;
  const float ratio = expf(lp - in.old_lp);
  const float rc = clampf(ratio, a.lo, a.hi);
  const float u = ratio * A;
  const float w = rc * A;
  const float su = u < w ? 1.0f : (u == w ? 0.5f : 0.0f);
  const float sw = w < u ? 1.0f : (u == w ? 0.5f : 0.0f);
  const float inr = (ratio >= a.lo && ratio <= a.hi) ? 1.0f : 0.0f;
  // d(policy_i)/d(ratio) = -A*(su + sw*inr); times 1/B (mean) and ratio (exp').
  o.g_lp = -(A * (su + sw * inr)) * a.inv_b * ratio;
  o.pol = -nan_min(u, w);

  const float d = in.v - in.ret;
  float dvl;
  if (a.use_vclip) {
    const float dv = in.v - in.vo;
    const float vcl = in.vo + clampf(dv, -a.vclip, a.vclip);
    const float d2 = vcl - in.ret;
    const float l1 = d * d;
    const float l2 = d2 * d2;
    o.vl = nan_max(l1, l2);
    const float s1 = l1 > l2 ? 1.0f : (l1 == l2 ? 0.5f : 0.0f);
    const float s2 = l2 > l1 ? 1.0f : (l1 == l2 ? 0.5f : 0.0f);
    const float in2 = (dv >= -a.vclip && dv <= a.vclip) ? 1.0f : 0.0f;
    dvl = s1 * (2.0f * d) + s2 * (2.0f * d2) * in2;
  } else {
    o.vl = d * d;
    dvl = 2.0f * d;
  }
  o.dval = a.vc * (dvl * a.inv_b);
  o.kl = in.old_lp - lp;
  o.clipped = fabsf(ratio - 1.0f) > a.clip ? 1.0f : 0.0f;
  return o;
}

// Categorical row: the A logits in zr[] (LDS or registers) are replaced by
// dloss/dlogits.  Softmax statistics in registers:
//   m = max z;  s = sum e_j, e_j = exp(z_j - m);  S = sum e_j (z_j - m)
//   log p_j = (z_j - m) - log s;   H = log s - S / s
//   dlogit_j = p_j * (ge * (z_j - m) + K) + 1[j == a] * g_lp,
//   K = ge * (H - log s) - g_lp,  ge = ec / B
// (ge * p_j * (log p_j + H) is the entropy term, -g_lp * p_j the log-prob
// term).  The per-logit exponentials use the hardware exp2 (one multiply by
// log2(e) and v_exp_f32, relative error ~1e-6 for |z_j - m| <= 20).  ai is
// the action index, -1 when outside [0, A) (the log-prob is then NaN).
// Returns the row's loss terms; H receives the row's entropy.
template <int MAXA, typename P>
__device__ __forceinline__ RowOut cat_row_grad(const P& a, float* zr, int A, int ai, float ge,
                                               const RowIn& in, float& H) {
  constexpr float kLog2e = 1.4426950408889634f;
  float t[MAXA], e[MAXA];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < MAXA; ++j)
    if (j < A) {
      t[j] = zr[j];
      m = fmaxf(m, t[j]);
    }
  float s = 0.0f, S = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXA; ++j)
    if (j < A) {
      const float tj = fmaxf(t[j] - m, -FLT_MAX);
      const float ej = __builtin_amdgcn_exp2f(tj * kLog2e);
      t[j] = tj;
      e[j] = ej;
      s += ej;
      S = fmaf(ej, tj, S);
    }
  const float log_s = logf(s);
  const float inv_s = 1.0f / s;
  H = log_s - S * inv_s;
  const float lp = ai >= 0 ? (zr[ai] - m) - log_s : __builtin_nanf("");
  const RowOut o = ppo_row_math(a, in, lp);
  const float K = ge * (H - log_s) - o.g_lp;
#pragma unroll
  for (int j = 0; j < MAXA; ++j)
    if (j < A) zr[j] = (e[j] * inv_s) * fmaf(ge, t[j], K);
  if (ai >= 0) zr[ai] += o.g_lp;
  return o;
}

}  // namespace ppo
