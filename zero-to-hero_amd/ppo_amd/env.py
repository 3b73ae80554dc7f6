"""CartPole-v1 for N environments on the GPU (ppo_cartpole_step).

The reference trains on gymnasium's CartPole-v1 (rl/deep/cli.py:179-180),
one transition per Python step (rl/deep/runner.py:56-74).  `CartPoleVec`
steps N copies in one launch with the same dynamics (csrc/cartpole.hip:
gymnasium CartPoleEnv's equations and constants, fp64 state, fp32
observations, termination at |x| > 2.4 or |theta| > 12 degrees, truncation
at 500 steps, reward 1 per step) and resets finished environments in the
same launch, so a whole rollout runs without the host touching the data.
gymnasium itself is not installed here: agreement with it is not tested, only
with the restated equations (oracle.cartpole_step_reference) and their
closed-form and symmetry properties.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .ops import _call, _require, _stream


class _Box:
    def __init__(self, shape: tuple) -> None:
        self.shape = shape


class _Discrete:
    def __init__(self, n: int) -> None:
        self.n = n


class CartPoleVec:
    """N independent CartPole-v1 environments on one GPU.

    `reset()` and `step(actions)` return device tensors that are overwritten
    by the next call (copy them to keep them): observations [N,4] fp32,
    rewards [N] fp32, dones [N] uint8 (terminated or truncated), terminated
    [N] uint8.  Reset states come from `generator` (seeded with `seed`).
    Completed episodes are tallied on the device: `episode_stats()` returns
    (number of completed episodes, mean return of those since the last
    call) and is the only method that synchronises.
    """

    observation_space = _Box((4,))
    action_space = _Discrete(2)

    def __init__(self, num_envs: int, device: str | torch.device = "cuda", seed: int = 24,
                 max_steps: int = 500) -> None:
        if num_envs < 1:
            raise ValueError(f"num_envs must be >= 1, got {num_envs}")
        if max_steps < 1:
            raise ValueError(f"max_steps must be >= 1, got {max_steps}")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("CartPoleVec runs on the GPU only (no CPU fallback)")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.num_envs, self.device, self.max_steps = num_envs, dev, max_steps
        N = num_envs
        self.state = torch.zeros(N, 4, dtype=torch.float64, device=dev)
        self.steps = torch.zeros(N, dtype=torch.int32, device=dev)
        self.obs = torch.zeros(N, 4, dtype=torch.float32, device=dev)
        self.rewards = torch.zeros(N, dtype=torch.float32, device=dev)
        self.dones = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.terminated = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.generator = torch.Generator(device=dev).manual_seed(seed)
        self._u = torch.empty(N, 4, dtype=torch.float32, device=dev)
        # per-environment episode tally, kept by the step kernel
        self._ret = torch.zeros(N, dtype=torch.float32, device=dev)
        self._done_sum = torch.zeros(N, dtype=torch.float64, device=dev)
        self._done_count = torch.zeros(N, dtype=torch.int32, device=dev)

    def reset(self) -> torch.Tensor:
        torch.rand(self.num_envs, 4, generator=self.generator, out=self._u)
        stream = _stream(self.device)
        _call("ppo_cartpole_reset", self.device, stream, self.state.data_ptr(),
              self.steps.data_ptr(), self._u.data_ptr(), self.obs.data_ptr(), self.num_envs,
              stream)
        self._ret.zero_()
        return self.obs

    def step(self, actions: torch.Tensor):
        self.step_into(actions, self.rewards, self.dones)
        return self.obs, self.rewards, self.dones, self.terminated

    def step_into(self, actions: torch.Tensor, rewards_out: torch.Tensor,
                  dones_out: torch.Tensor,
                  reset_uniforms: Optional[torch.Tensor] = None) -> torch.Tensor:
        """step() writing the rewards and dones into the given [N] tensors
        (e.g. row t of a RolloutBuffer) instead of the environment's own;
        returns the observations.  `reset_uniforms` [N,4] U[0,1) replaces the
        environment's own draw (no random launch: for graph capture)."""
        _require(actions, "actions", (torch.int32,), self.device)
        if actions.shape != (self.num_envs,):
            raise ValueError(f"actions must be [N]=[{self.num_envs}], got {tuple(actions.shape)}")
        _require(rewards_out, "rewards_out", (torch.float32,), self.device)
        _require(dones_out, "dones_out", (torch.uint8,), self.device)
        if rewards_out.numel() != self.num_envs or dones_out.numel() != self.num_envs:
            raise ValueError("rewards_out and dones_out must hold N values")
        if reset_uniforms is None:
            torch.rand(self.num_envs, 4, generator=self.generator, out=self._u)
            reset_uniforms = self._u
        else:
            _require(reset_uniforms, "reset_uniforms", (torch.float32,), self.device)
            if reset_uniforms.numel() != self.num_envs * 4:
                raise ValueError("reset_uniforms must hold N x 4 values")
        stream = _stream(self.device)
        _call("ppo_cartpole_step", self.device, stream, self.state.data_ptr(),
              self.steps.data_ptr(), actions.data_ptr(), reset_uniforms.data_ptr(),
              self.max_steps,
              self.obs.data_ptr(), rewards_out.data_ptr(), dones_out.data_ptr(),
              self.terminated.data_ptr(), self._ret.data_ptr(), self._done_sum.data_ptr(),
              self._done_count.data_ptr(), self.num_envs, stream)
        return self.obs

    def episode_stats(self) -> tuple[int, float]:
        """(completed episodes, their mean return) since the last call."""
        count = int(self._done_count.sum().item())
        total = float(self._done_sum.sum().item())
        self._done_sum.zero_()
        self._done_count.zero_()
        return count, (total / count if count else float("nan"))
