"""ppo_amd — the PPO update path of mrhooray/zero-to-hero (rl/deep) on MI355X.

Hand-written HIP kernels for gfx950 (libppo_amd.so, C ABI in
include/ppo_amd.h) behind the reference's own PPO surface:

  ops       gae, gae_normalize, normalize_advantages, discounted_returns,
            gather_rows, sample_categorical, sample_gaussian,
            ppo_loss_discrete, ppo_loss_gaussian (+ *_fused functional forms)
  agent     PPOAgent, PPOConfig, TrainingConfig, MLP, Transition,
            RolloutStep, PendingStep, cartpole_sizes — rl/deep/agents/ppo.py
            and common.py, same names and signatures
  rollout   RolloutBuffer ([T,N] env-contiguous, on device) and VecPPO
  optim     ClippedAdam (clip_grad_norm_ + Adam, two launches)
  reference_patch  _advantages / _update_batch for the reference's own
            PPOAgent class (reference_patch.apply(PPOAgent))
  torch_ops the hot path as registered operators, torch.ops.ppo_amd.*
            (gae, gae_normalize, normalize_advantages, ppo_loss_discrete,
            ppo_loss_gaussian), visible to torch.compile and the dispatcher
"""

from . import _lib, reference_patch
from .agent import (
    MLP,
    PendingStep,
    PPOAgent,
    PPOConfig,
    RolloutStep,
    TrainingConfig,
    Transition,
    cartpole_sizes,
)
from .ops import (
    LossStats,
    discounted_returns,
    gae,
    gather_rows,
    gae_normalize,
    check_waits,
    mlp_act_categorical,
    mlp_forward_categorical,
    mlp_fusable,
    normalize_advantages,
    ppo_loss_discrete,
    ppo_loss_discrete_fused,
    ppo_loss_gaussian,
    ppo_loss_gaussian_fused,
    ppo_mlp_cat_grads,
    ppo_mlp_cat_step,
    sample_categorical,
    sample_gaussian,
)
from . import torch_ops  # registers torch.ops.ppo_amd.*
from .env import CartPoleVec
from .optim import ClippedAdam
from .rollout import RolloutBuffer, VecPPO

LIB_PATH = _lib.LIB_PATH


def load_library():
    """Load libppo_amd.so (raises if it is not built)."""
    return _lib.load()


__all__ = [
    "CartPoleVec",
    "ClippedAdam",
    "LIB_PATH",
    "LossStats",
    "MLP",
    "PPOAgent",
    "PPOConfig",
    "PendingStep",
    "RolloutBuffer",
    "RolloutStep",
    "TrainingConfig",
    "Transition",
    "VecPPO",
    "cartpole_sizes",
    "check_waits",
    "discounted_returns",
    "gae",
    "gae_normalize",
    "gather_rows",
    "load_library",
    "mlp_act_categorical",
    "mlp_forward_categorical",
    "mlp_fusable",
    "reference_patch",
    "normalize_advantages",
    "ppo_loss_discrete",
    "ppo_loss_discrete_fused",
    "ppo_loss_gaussian",
    "ppo_loss_gaussian_fused",
    "ppo_mlp_cat_grads",
    "ppo_mlp_cat_step",
    "sample_categorical",
    "sample_gaussian",
]
