"""The hot path as registered torch operators: torch.ops.ppo_amd.*.

Each operator runs the same HIP kernels as the functions in ops.py (it calls
them), but through torch's dispatcher, so it is visible to torch.compile
(with the fake implementations below, a compiled function traces through it
without a graph break), to torch.library.opcheck and to the profiler's op
view.  The implementations are registered for CUDA (HIP) tensors only: a CPU
tensor raises NotImplementedError, as there is no CPU fallback.

  ppo_amd::gae(rewards, values, dones, last_value?, gamma, lam) -> (adv, ret)
      PPOAgent._advantages + returns (rl/deep/agents/ppo.py:123-124, 173-193)
  ppo_amd::gae_normalize(rewards, values, dones, last_value?, gamma, lam, eps)
      -> (adv, ret, adv_n, stats[2])        ... plus ppo.py:126-127, fused
  ppo_amd::normalize_advantages(adv, eps) -> adv_n      (ppo.py:126-127)
  ppo_amd::ppo_loss_discrete(logits, actions, old_log_probs, advantages,
      returns, values, old_values?, clip_ratio, vf_clip?, value_coef,
      entropy_coef) -> (scalars[6], dlogits, dvalues)   (ppo.py:150-169)
  ppo_amd::ppo_loss_gaussian(mu, log_std, actions, old_log_probs, advantages,
      returns, values, old_values?, clip_ratio, vf_clip?, value_coef,
      entropy_coef) -> (scalars[6], dmu, dlog_std, dvalues)

The loss operators are differentiable in their first output: backward of
scalars[0] (the total loss; the other scalars are reported values) scales the
fused kernel's gradients by the incoming gradient, as ops.ppo_loss_discrete
does.  Their gradient outputs are marked non-differentiable.
"""

from typing import Optional

import torch
from torch import Tensor

from . import _lib, ops

_NS = "ppo_amd"


def _scalars_like(t: Tensor) -> Tensor:
    return torch.empty(_lib.PPO_NUM_SCALARS, dtype=torch.float32, device=t.device)


# ---------------------------------------------------------------------------
# GAE and normalisation
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::gae", mutates_args=(), device_types="cuda")
def gae(rewards: Tensor, values: Tensor, dones: Tensor, last_value: Optional[Tensor],
        gamma: float, lam: float) -> tuple[Tensor, Tensor]:
    adv, ret = ops.gae(rewards, values, dones, last_value, gamma, lam)
    return adv, ret


@gae.register_fake
def _gae_fake(rewards, values, dones, last_value, gamma, lam):
    return torch.empty_like(rewards), torch.empty_like(rewards)


@torch.library.custom_op(f"{_NS}::gae_normalize", mutates_args=(), device_types="cuda")
def gae_normalize(rewards: Tensor, values: Tensor, dones: Tensor, last_value: Optional[Tensor],
                  gamma: float, lam: float, eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    adv, ret, adv_n, stats = ops.gae_normalize(rewards, values, dones, last_value, gamma, lam,
                                               eps, return_stats=True)
    return adv, ret, adv_n, stats


@gae_normalize.register_fake
def _gae_normalize_fake(rewards, values, dones, last_value, gamma, lam, eps):
    return (torch.empty_like(rewards), torch.empty_like(rewards), torch.empty_like(rewards),
            torch.empty(2, dtype=torch.float32, device=rewards.device))


@torch.library.custom_op(f"{_NS}::normalize_advantages", mutates_args=(), device_types="cuda")
def normalize_advantages(advantages: Tensor, eps: float) -> Tensor:
    return ops.normalize_advantages(advantages, eps)


@normalize_advantages.register_fake
def _normalize_advantages_fake(advantages, eps):
    return torch.empty_like(advantages)


# ---------------------------------------------------------------------------
# Fused PPO losses (forward + backward in one launch)
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::ppo_loss_discrete", mutates_args=(), device_types="cuda")
def ppo_loss_discrete(logits: Tensor, actions: Tensor, old_log_probs: Tensor, advantages: Tensor,
                      returns: Tensor, values: Tensor, old_values: Optional[Tensor],
                      clip_ratio: float, vf_clip: Optional[float], value_coef: float,
                      entropy_coef: float) -> tuple[Tensor, Tensor, Tensor]:
    return ops.ppo_loss_discrete_fused(logits, actions, old_log_probs, advantages, returns,
                                       values, old_values, clip_ratio, vf_clip, value_coef,
                                       entropy_coef)


@ppo_loss_discrete.register_fake
def _ppo_loss_discrete_fake(logits, actions, old_log_probs, advantages, returns, values,
                            old_values, clip_ratio, vf_clip, value_coef, entropy_coef):
    return _scalars_like(logits), torch.empty_like(logits), torch.empty_like(values)


def _discrete_setup(ctx, inputs, output):
    _, dlogits, dvalues = output
    ctx.mark_non_differentiable(dlogits, dvalues)
    ctx.save_for_backward(dlogits, dvalues)


def _discrete_backward(ctx, grad_scalars, grad_dlogits, grad_dvalues):
    dlogits, dvalues = ctx.saved_tensors
    g = grad_scalars[0]
    return dlogits * g, None, None, None, None, dvalues * g, None, None, None, None, None


ppo_loss_discrete.register_autograd(_discrete_backward, setup_context=_discrete_setup)


@torch.library.custom_op(f"{_NS}::ppo_loss_gaussian", mutates_args=(), device_types="cuda")
def ppo_loss_gaussian(mu: Tensor, log_std: Tensor, actions: Tensor, old_log_probs: Tensor,
                      advantages: Tensor, returns: Tensor, values: Tensor,
                      old_values: Optional[Tensor], clip_ratio: float, vf_clip: Optional[float],
                      value_coef: float, entropy_coef: float
                      ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return ops.ppo_loss_gaussian_fused(mu, log_std, actions, old_log_probs, advantages, returns,
                                       values, old_values, clip_ratio, vf_clip, value_coef,
                                       entropy_coef)


@ppo_loss_gaussian.register_fake
def _ppo_loss_gaussian_fake(mu, log_std, actions, old_log_probs, advantages, returns, values,
                            old_values, clip_ratio, vf_clip, value_coef, entropy_coef):
    return (_scalars_like(mu), torch.empty_like(mu), torch.empty_like(log_std),
            torch.empty_like(values))


def _gaussian_setup(ctx, inputs, output):
    _, dmu, dlog_std, dvalues = output
    ctx.mark_non_differentiable(dmu, dlog_std, dvalues)
    ctx.save_for_backward(dmu, dlog_std, dvalues)


def _gaussian_backward(ctx, grad_scalars, grad_dmu, grad_dlog_std, grad_dvalues):
    dmu, dlog_std, dvalues = ctx.saved_tensors
    g = grad_scalars[0]
    return (dmu * g, dlog_std * g, None, None, None, None, dvalues * g, None, None, None, None,
            None)


ppo_loss_gaussian.register_autograd(_gaussian_backward, setup_context=_gaussian_setup)
