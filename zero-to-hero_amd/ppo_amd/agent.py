"""PPO agent whose update runs on the MI355X kernels.

Mirrors the reference module rl/deep/agents/ppo.py (and the pieces of
rl/deep/agents/common.py and rl/deep/type.py it uses) name for name, with the
same method signatures, so that a caller of the reference's PPOAgent can use
this one unchanged.  Differences, all on the device side:
  * `_advantages` runs the GAE kernel (fp64 recurrence, the reference's
    operation order) instead of a Python loop;
  * `_update` normalises with the fused normalisation kernel;
  * `_update_batch` computes the loss and its gradient with the fused loss
    kernel; the MLPs, clip_grad_norm_ and Adam stay in torch on the GPU.
The environment is duck-typed (anything with observation_space.shape and
action_space.n), since gymnasium is not a dependency here.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch
from torch import nn
from torch.distributions import Categorical

from . import ops


# ---------------------------------------------------------------------------
# Configuration (rl/deep/type.py:30-41, rl/deep/agents/ppo.py:15-22)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class TrainingConfig:
    """Same fields and defaults as rl/deep/type.py:30-41."""

    gamma: float = 0.99
    lr: float = 3e-4
    seed: int = 24
    hidden_size: int = 128
    debug: bool = False
    batch_size: int = 128
    replay_size: int = 1024 * 16
    warmup_steps: int = 1024 * 2


@dataclass(frozen=True)
class PPOConfig:
    """rl/deep/agents/ppo.py:15-22, plus value clipping (None = the
    reference's plain mse value loss)."""

    epochs: int = 4
    clip_ratio: float = 0.2
    gae_lambda: float = 0.95
    value_coef: float = 0.5
    entropy_coef: float = 0.01
    gradient_clip: float = 0.5
    vf_clip: Optional[float] = None


# ---------------------------------------------------------------------------
# Models and rollout records (rl/deep/agents/common.py:16-39, ppo.py:25-35)
# ---------------------------------------------------------------------------
class MLP(nn.Module):
    """Linear-act-Linear-act-Linear, rl/deep/agents/common.py:16-28.  The
    reference uses ReLU; `activation="tanh"` gives the benchmark's 4-64-64 tanh
    variant."""

    def __init__(self, input_size: int, hidden_size: int, output_size: int,
                 activation: str = "relu") -> None:
        super().__init__()
        act = {"relu": nn.ReLU, "tanh": nn.Tanh}[activation]
        self.net = nn.Sequential(
            nn.Linear(input_size, hidden_size),
            act(),
            nn.Linear(hidden_size, hidden_size),
            act(),
            nn.Linear(hidden_size, output_size),
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x)


@dataclass(frozen=True)
class Transition:
    """rl/deep/agents/common.py:31-39."""

    observation: np.ndarray
    action: int
    reward: float
    next_observation: np.ndarray
    terminated: bool
    truncated: bool


@dataclass(frozen=True)
class RolloutStep:
    """ppo.py:25-29."""

    transition: Transition
    log_prob: torch.Tensor
    value: torch.Tensor


@dataclass(frozen=True)
class PendingStep:
    """ppo.py:32-35."""

    log_prob: torch.Tensor
    value: torch.Tensor


def cartpole_sizes(env) -> tuple[int, int]:
    """rl/deep/agents/common.py:82-87 for duck-typed spaces: a Box-like
    observation space (has .shape) and a Discrete-like action space (has .n);
    TypeError otherwise, as the reference raises."""
    obs_space = getattr(env, "observation_space", None)
    act_space = getattr(env, "action_space", None)
    if obs_space is None or getattr(obs_space, "shape", None) is None:
        raise TypeError("CartPole agents require a Box observation space")
    if act_space is None or getattr(act_space, "n", None) is None:
        raise TypeError("CartPole agents require a Discrete action space")
    return int(np.prod(obs_space.shape)), int(act_space.n)


# ---------------------------------------------------------------------------
# The agent (rl/deep/agents/ppo.py:38-193)
# ---------------------------------------------------------------------------
class PPOAgent:
    name = "ppo"

    def __init__(
        self,
        env,
        config: TrainingConfig,
        ppo_config: PPOConfig = PPOConfig(),
        device: str | torch.device = "cuda",
        activation: str = "relu",
    ) -> None:
        torch.manual_seed(config.seed)                                    # ppo.py:47

        self.config = config
        self.ppo_config = ppo_config
        self.device = torch.device(device)
        observation_size, action_count = cartpole_sizes(env)

        # initialised on the CPU generator exactly as the reference does, then
        # moved, so both start from identical weights for one seed
        self.policy = MLP(observation_size, config.hidden_size, action_count, activation)
        self.value = MLP(observation_size, config.hidden_size, 1, activation)
        self.policy.to(self.device)
        self.value.to(self.device)
        self.parameters = list(self.policy.parameters()) + list(self.value.parameters())
        self.optimizer = torch.optim.Adam(self.parameters, lr=config.lr)

        self.rollout: list[RolloutStep] = []
        self.pending_step: PendingStep | None = None

    def start_episode(self, episode: int) -> None:
        self.rollout = []
        self.pending_step = None

    @torch.no_grad()
    def select_action(self, observation: np.ndarray, training: bool = True) -> int:
        """ppo.py:65-79.  The policy runs on the device; sampling uses a CPU
        Categorical so the global CPU generator is consumed as in the
        reference.  log_prob and value are 0-d CPU tensors, as there."""
        obs = torch.as_tensor(observation, dtype=torch.float32, device=self.device)
        logits = self.policy(obs).cpu()
        if not training:
            return int(torch.argmax(logits).item())

        distribution = Categorical(logits=logits)
        action = distribution.sample()
        self.pending_step = PendingStep(
            log_prob=distribution.log_prob(action),
            value=self.value(obs).squeeze().cpu(),
        )
        return int(action.item())

    def update(
        self,
        observation: np.ndarray,
        action: int,
        reward: float,
        next_observation: np.ndarray,
        terminated: bool,
        truncated: bool,
    ) -> None:
        """ppo.py:81-107."""
        if self.pending_step is None:
            return

        self.rollout.append(
            RolloutStep(
                transition=Transition(
                    observation=observation,
                    action=action,
                    reward=reward,
                    next_observation=next_observation,
                    terminated=terminated,
                    truncated=truncated,
                ),
                log_prob=self.pending_step.log_prob,
                value=self.pending_step.value,
            )
        )
        self.pending_step = None

    def end_episode(self) -> None:
        if self.rollout:
            self._update()

    def _update(self) -> None:
        """ppo.py:113-139 with the GAE, normalisation and loss on the GPU.
        The permutation comes from torch.randperm on the global CPU
        generator, as at :130, so the minibatch index stream is the
        reference's bit for bit."""
        dev = self.device
        observations = torch.as_tensor(
            np.array([step.transition.observation for step in self.rollout]),
            dtype=torch.float32,
        ).to(dev)
        actions_host = torch.as_tensor(
            [step.transition.action for step in self.rollout], dtype=torch.int64
        )
        action_count = self.policy.net[-1].out_features
        # checked on the host copy (no device synchronisation); torch.
        # distributions' support check raises this inside :151
        if bool(((actions_host < 0) | (actions_host >= action_count)).any()):
            raise ValueError(
                "The value argument must be within the support of the categorical "
                f"distribution (actions in [0, {action_count}))"
            )
        actions = actions_host.to(dev)
        old_log_probs = torch.stack([step.log_prob for step in self.rollout]).to(dev)
        old_values = torch.stack([step.value for step in self.rollout]).to(
            device=dev, dtype=torch.float32
        )
        advantages = self._advantages(old_values)
        returns = advantages + old_values

        if len(advantages) > 1:
            advantages = ops.normalize_advantages(advantages)

        for _ in range(self.ppo_config.epochs):
            indices = torch.randperm(len(actions))
            for start in range(0, len(actions), self.config.batch_size):
                batch_indices = indices[start : start + self.config.batch_size].to(dev)
                extra = {}
                if self.ppo_config.vf_clip is not None:
                    # the clipped value loss needs the rollout's values
                    extra["old_values"] = old_values[batch_indices]
                self._update_batch(
                    observations[batch_indices],
                    actions[batch_indices],
                    old_log_probs[batch_indices],
                    advantages[batch_indices],
                    returns[batch_indices],
                    **extra,
                )

    def _update_batch(
        self,
        observations: torch.Tensor,
        actions: torch.Tensor,
        old_log_probs: torch.Tensor,
        advantages: torch.Tensor,
        returns: torch.Tensor,
        old_values: Optional[torch.Tensor] = None,
    ) -> None:
        """ppo.py:141-171: MLP forwards in torch, the fused loss kernel for
        the loss and its gradient, then backward through the MLPs,
        clip_grad_norm_ and Adam.  `old_values` (the rollout's values of the
        minibatch rows) is needed only with PPOConfig.vf_clip, which the
        reference does not have; ValueError if it is missing then."""
        if self.ppo_config.vf_clip is not None and old_values is None:
            raise ValueError("PPOConfig.vf_clip needs the minibatch's old_values")
        logits = self.policy(observations)
        values = self.value(observations).squeeze(1)
        loss, _ = ops.ppo_loss_discrete(
            logits.contiguous(),
            actions.contiguous(),
            old_log_probs.contiguous(),
            advantages.contiguous(),
            returns.contiguous(),
            values.contiguous(),
            clip_ratio=self.ppo_config.clip_ratio,
            vf_clip=self.ppo_config.vf_clip,
            value_coef=self.ppo_config.value_coef,
            entropy_coef=self.ppo_config.entropy_coef,
            old_values=None if old_values is None else old_values.contiguous(),
        )
        self.optimizer.zero_grad()
        loss.backward()
        nn.utils.clip_grad_norm_(self.parameters, self.ppo_config.gradient_clip)
        self.optimizer.step()

    def _advantages(self, values: torch.Tensor) -> torch.Tensor:
        """ppo.py:173-193 on the GPU: one env, no bootstrap, `terminated or
        truncated` as the done flag.  Returns fp32 advantages on the device.

        The recurrence runs in fp64 in the reference's operation order, but
        the rewards enter as fp32 (the kernel's rollout layout): a reward that
        fp32 represents exactly (CartPole's 1.0, any integer, any multiple of
        a power of two) gives the reference's advantages bit for bit; any
        other reward r is off by at most |r| * 2^-24, so an advantage moves by
        at most max|r| * 2^-24 / (1 - gamma * lambda), i.e. relative ~1e-6
        for gamma = 0.99, lambda = 0.95 (tests/test_gpu_agent.py checks the
        bound with rewards of 0.1)."""
        rewards = torch.tensor(
            [step.transition.reward for step in self.rollout], dtype=torch.float32
        )
        dones = torch.tensor(
            [bool(step.transition.terminated or step.transition.truncated)
             for step in self.rollout],
            dtype=torch.uint8,
        )
        v = values.to(device=self.device, dtype=torch.float32).contiguous()
        adv, _ = ops.gae(
            rewards.to(self.device), v, dones.to(self.device), None,
            self.config.gamma, self.ppo_config.gae_lambda,
        )
        return adv
