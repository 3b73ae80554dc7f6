"""Method patches for the reference's own PPOAgent (rl/deep/agents/ppo.py).

For a maintainer who keeps the reference class and swaps only its hot
functions.  The reference agent keeps its networks, its rollout and its
optimizer on the CPU; these methods move the tensors they hand to the
kernels to the GPU and bring back what the reference's code reads next:

    from deep.agents.ppo import PPOAgent
    from ppo_amd import reference_patch
    reference_patch.apply(PPOAgent)

  _advantages    ppo.py:173-193 on the GPU (GAE kernel, fp64 recurrence in
                 the reference's operation order); returns CPU fp32
                 advantages, so ppo.py:123-127 run unchanged on the CPU
  _update_batch  ppo.py:141-171 with the loss and its gradient from the
                 fused loss kernel: the CPU networks' logits and values go to
                 the GPU through `.to("cuda")`, whose backward brings the
                 gradient back to the CPU parameters; clip_grad_norm_ and
                 Adam stay the reference's.
"""

from __future__ import annotations

import torch
from torch import nn

from . import ops


def _advantages(self, values: torch.Tensor) -> torch.Tensor:
    """ppo.py:173-193: `values` [T] (CPU), rewards and done flags from
    self.rollout; returns the advantages as a CPU fp32 tensor [T]."""
    steps = self.rollout
    rewards = torch.tensor([s.transition.reward for s in steps], dtype=torch.float32)
    dones = torch.tensor([bool(s.transition.terminated or s.transition.truncated)
                          for s in steps], dtype=torch.uint8)
    adv, _ = ops.gae(rewards.cuda(), values.to(torch.float32).cuda(), dones.cuda(), None,
                     self.config.gamma, self.ppo_config.gae_lambda)
    return adv.cpu()


def _update_batch(self, observations: torch.Tensor, actions: torch.Tensor,
                  old_log_probs: torch.Tensor, advantages: torch.Tensor,
                  returns: torch.Tensor) -> None:
    """ppo.py:141-171 with ops.ppo_loss_discrete for :150-167."""
    logits = self.policy(observations)
    values = self.value(observations).squeeze(1)
    loss, _ = ops.ppo_loss_discrete(
        logits.cuda().contiguous(), actions.cuda().contiguous(),
        old_log_probs.cuda().contiguous(), advantages.cuda().contiguous(),
        returns.cuda().contiguous(), values.cuda().contiguous(),
        clip_ratio=self.ppo_config.clip_ratio, value_coef=self.ppo_config.value_coef,
        entropy_coef=self.ppo_config.entropy_coef)
    self.optimizer.zero_grad()
    loss.backward()
    nn.utils.clip_grad_norm_(self.parameters, self.ppo_config.gradient_clip)
    self.optimizer.step()


def apply(agent_class: type) -> type:
    """Installs both methods on `agent_class` (the reference's PPOAgent)."""
    agent_class._advantages = _advantages
    agent_class._update_batch = _update_batch
    return agent_class
