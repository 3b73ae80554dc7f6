"""PPO agent whose update runs on the MI355X kernels.

Mirrors the reference module rl/deep/agents/ppo.py (and the pieces of
rl/deep/agents/common.py and rl/deep/type.py it uses) name for name, with the
same method signatures, so that a caller of the reference's PPOAgent can use
this one unchanged.  Differences, all on the device side:
  * `_advantages` runs the GAE kernel (fp64 recurrence, the reference's
    operation order) instead of a Python loop;
  * `_update` normalises with the fused normalisation kernel;
  * when the networks are MLPs the fused kernels support (the reference's
    own 4-128-128 ReLU networks are), `_update` runs every minibatch as the
    fused MLP step (gather + both forwards + loss + backward, then the
    gradient reduction with clip_grad_norm_ and Adam: two launches), with the
    permutations of all epochs uploaded in one copy, and replays the
    minibatch loop from HIP graphs when an episode has the previous one's
    length; `optimizer` is then a ClippedAdam (clip + Adam fused);
  * otherwise `_update_batch` computes the loss and its gradient with the
    fused loss kernel and the MLPs, clip_grad_norm_ and Adam stay in torch;
  * `select_action` brings the logits and the value to the host in one copy
    (one forward launch for both networks when fused) and draws the action
    with the operations of a Categorical, not the distribution object.
The environment is duck-typed (anything with observation_space.shape and
action_space.n), since gymnasium is not a dependency here.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch
from torch import nn

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


def sample_categorical(logits: torch.Tensor) -> tuple[int, torch.Tensor]:
    """Categorical(logits=logits).sample() and .log_prob() of that sample, as
    ppo.py:72-78 uses them, for one CPU row of logits [A]: the operations
    torch.distributions.Categorical runs (normalise by logsumexp, softmax,
    one torch.multinomial draw with replacement on the global generator,
    gather of the normalised logit), without building the distribution
    object, whose construction costs more than the draw.  Same action, same
    log-probability bits and same generator state as the distribution for
    the same logits.  Returns (action, 0-d log-probability tensor).  NaN
    logits raise ValueError, as the distribution's argument validation does
    (checked only once the draw has failed on them)."""
    normalized = logits - logits.logsumexp(-1, keepdim=True)
    try:
        drawn = torch.multinomial(torch.softmax(normalized, -1).reshape(1, -1), 1, True)
    except RuntimeError:
        if bool(torch.isnan(logits).any()):
            raise ValueError("Expected parameter logits to satisfy the constraint "
                             f"IndependentConstraint(Real(), 1), but found invalid values:\n{logits}")
        raise
    action = int(drawn[0, 0])
    return action, normalized[action].clone()


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
    """rl/deep/agents/ppo.py:38-193 with the update on the GPU.

    `fused_update` (default: whenever ops.mlp_fusable accepts the networks)
    takes the fused minibatch step described in the module docstring;
    `graphs` (default True) lets the fused loop replay captured graphs for
    episodes of a length seen in the previous update.  Both follow the
    reference's randomness: actions are drawn as a CPU Categorical draws them
    (sample_categorical) and the minibatches come from torch.randperm, both on the global CPU generator,
    so one seed gives the reference's trajectories and index stream."""

    name = "ppo"

    def __init__(
        self,
        env,
        config: TrainingConfig,
        ppo_config: PPOConfig = PPOConfig(),
        device: str | torch.device = "cuda",
        activation: str = "relu",
        fused_update: Optional[bool] = None,
        graphs: bool = True,
    ) -> None:
        torch.manual_seed(config.seed)                                    # ppo.py:47

        self.config = config
        self.ppo_config = ppo_config
        self.device = torch.device(device)
        observation_size, action_count = cartpole_sizes(env)
        self.action_count = action_count

        # initialised on the CPU generator exactly as the reference does, then
        # moved, so both start from identical weights for one seed
        self.policy = MLP(observation_size, config.hidden_size, action_count, activation)
        self.value = MLP(observation_size, config.hidden_size, 1, activation)
        self.policy.to(self.device)
        self.value.to(self.device)
        self.parameters = list(self.policy.parameters()) + list(self.value.parameters())
        fusable = ops.mlp_fusable(self.policy, self.value)
        if fused_update and not fusable:
            raise ValueError("fused_update needs MLPs on the GPU that ops.mlp_fusable accepts")
        self.fused_update = fusable if fused_update is None else bool(fused_update)
        self._fused_act = fusable
        self._vec = None
        if self.fused_update:
            from .rollout import VecPPO

            self._vec = VecPPO(self.policy, self.value, ppo_config, gamma=config.gamma,
                               lr=config.lr, batch_size=config.batch_size, fused_update=True,
                               graphs=graphs, fused_mlp=True)
            self.optimizer = self._vec.optimizer
            # (the reference's update is synchronous: report a give-up at once)
            self._vec.check_waits = "sync"
        else:
            self.optimizer = torch.optim.Adam(self.parameters, lr=config.lr)
        self.graphs = graphs
        self._stage: dict = {}  # rollout length -> persistent device arrays (graph replays)
        self._host: Optional[torch.Tensor] = None  # pinned staging buffer of _upload_rollout
        self._host_ready = None  # event: the last upload has read _host
        self._last_n = -1
        self._act_ctx = None  # select_action's launch arguments and pinned buffer
        self._act_ids: tuple = ()
        self._act_ok = False

        self.rollout: list[RolloutStep] = []
        self.pending_step: PendingStep | None = None

    def start_episode(self, episode: int) -> None:
        self.rollout = []
        self.pending_step = None

    @torch.no_grad()
    def select_action(self, observation: np.ndarray, training: bool = True) -> int:
        """ppo.py:65-79.  The networks run on the device and the logits and
        the value come back to the host in one copy; the action is drawn with
        a Categorical's operations on the host (sample_categorical), so the
        global CPU generator is consumed as in the reference.  log_prob and value are 0-d CPU tensors, as there."""
        A = self.action_count
        if self._fused_act and np.ndim(observation) == 1 and self._act_ready():
            logits, value = self._forward_pinned(observation)
        else:
            obs = torch.as_tensor(observation, dtype=torch.float32).to(self.device)
            host = torch.cat([self.policy(obs).reshape(-1), self.value(obs).reshape(-1)]).cpu()
            logits, value = host[:A], host[A]
        if not training:
            return int(torch.argmax(logits).item())

        action, log_prob = sample_categorical(logits)
        self.pending_step = PendingStep(log_prob=log_prob, value=value)
        return action

    def _act_ready(self) -> bool:
        """The networks are still ones the fused forward runs (checked again
        only when a network object was replaced)."""
        ids = (id(self.policy), id(self.value))
        if self._act_ids != ids:
            self._act_ids = ids
            self._act_ok = ops.mlp_fusable(self.policy, self.value)
        return self._act_ok

    def _forward_pinned(self, observation) -> tuple[torch.Tensor, torch.Tensor]:
        """Both networks on one observation through ppo_mlp_forward_cat_f32,
        reading it from and writing the logits and value to pinned host
        memory (no copy launches), then one stream synchronisation.  The
        launch arguments are built once and rebuilt when a network or its
        parameter storage changes."""
        key = (id(self.policy), id(self.value),
               tuple(p.data_ptr() for p in self.parameters))
        if self._act_ctx is None or self._act_ctx[0] != key:
            from . import _lib

            lp, act = ops.mlp_structure(self.policy)
            lv, _ = ops.mlp_structure(self.value)
            D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
            structs = (_lib.Mlp3(), _lib.Mlp3())
            for st, layers in zip(structs, (lp, lv)):
                for i, m in enumerate(layers):
                    st.weight[i] = m.weight.data_ptr()
                    st.bias[i] = m.bias.data_ptr()
            io = torch.zeros(D + A + 1, dtype=torch.float32, pin_memory=True)
            ptr = io.data_ptr()
            head = (ctypes.byref(structs[0]), ctypes.byref(structs[1]), D, H, A,
                    _lib.PPO_ACT_TANH if act == "tanh" else _lib.PPO_ACT_RELU, ptr, 1,
                    ptr + 4 * D, ptr + 4 * (D + A))
            self._act_ctx = (key, structs, io, io.numpy(), head, D, A,
                             _lib.load().ppo_mlp_forward_cat_f32)
        _, _, io, io_np, head, D, A, fn = self._act_ctx
        io_np[:D] = observation
        stream = torch.cuda.current_stream(self.device)
        code = fn(*head, stream.cuda_stream)
        if code:
            from . import _lib

            _lib.check("ppo_mlp_forward_cat_f32", code)
        stream.synchronize()
        out = torch.from_numpy(io_np[D:].copy())
        return out[:A], out[A]

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
        reference's bit for bit.  The rollout's arrays reach the device in
        one copy (_upload_rollout)."""
        dev = self.device
        staged = self._upload_rollout()
        observations, actions = staged["obs"], staged["act"]
        old_log_probs, old_values = staged["lp"], staged["val"]
        fused = self.fused_update and "_update_batch" not in self.__dict__ and (
            type(self)._update_batch is PPOAgent._update_batch)
        if fused and "_advantages" not in self.__dict__ and (
                type(self)._advantages is PPOAgent._advantages):
            # :123-127 in one launch: advantages, returns = advantages +
            # old_values, and the normalised advantages written over the raw
            # ones (the identity for a single step, as the :126 guard)
            advantages, returns, _ = ops.gae_normalize(
                staged["rew"], old_values, staged["done"], None, self.config.gamma,
                self.ppo_config.gae_lambda, out=(staged["adv"], staged["ret"]), keep_raw=False)
        else:
            advantages = self._advantages(old_values)
            returns = advantages + old_values
            if len(advantages) > 1:
                advantages = ops.normalize_advantages(advantages)

        # The fused loop stands in for the minibatch loop below unless
        # _update_batch was replaced (a subclass or an instance attribute),
        # in which case that method is what must run per minibatch.
        if fused:
            self._update_fused(staged, advantages, returns)
            return

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
        if dev.type == "cuda":
            ops.check_waits(dev)

    def _upload_rollout(self) -> dict:
        """The rollout's observations [n,D] fp32, actions [n] int64, old
        log-probabilities, old values and rewards [n] fp32 and done flags
        (terminated or truncated) [n] uint8, written into one pinned host
        buffer and copied to the device in one transfer (ppo.py:114-122, and
        the rewards and flags :173-193 reads), into device arrays kept per
        rollout length (the two most recent lengths), with room for the
        advantages and returns: a repeated length reuses the addresses its
        captured graphs read.  Out-of-range actions raise ValueError here,
        checked on the host (torch.distributions' support check raises it
        inside :151)."""
        steps = self.rollout
        n = len(steps)
        D = int(np.asarray(steps[0].transition.observation).size) if n else 0
        # byte offsets of the arrays, each 16-byte aligned
        sizes = (("obs", n * D * 4), ("lp", n * 4), ("val", n * 4), ("rew", n * 4),
                 ("act", n * 8), ("done", n))
        offsets, nbytes = {}, 0
        for name, size in sizes:
            offsets[name] = nbytes
            nbytes += (size + 15) // 16 * 16
        if self._host is None or self._host.numel() < nbytes:
            self._host = torch.empty(max(nbytes, 2 * (0 if self._host is None else
                                                          self._host.numel())),
                                     dtype=torch.uint8, pin_memory=self.device.type == "cuda")
        elif self._host_ready is not None:
            self._host_ready.synchronize()  # the previous upload has read the buffer

        def views(buf):
            def f32(name, *shape):
                o = offsets[name]
                return buf[o : o + 4 * int(np.prod(shape))].view(torch.float32).view(*shape)

            return {"obs": f32("obs", n, D), "lp": f32("lp", n), "val": f32("val", n),
                    "rew": f32("rew", n),
                    "act": buf[offsets["act"] : offsets["act"] + 8 * n].view(torch.int64),
                    "done": buf[offsets["done"] : offsets["done"] + n]}

        host = views(self._host)
        if n:
            np.stack([s.transition.observation for s in steps], out=host["obs"].numpy(),
                     casting="unsafe")
        acts = host["act"].numpy()
        acts[:] = [s.transition.action for s in steps]
        A = self.policy.net[-1].out_features
        if n and (acts.min() < 0 or acts.max() >= A):
            raise ValueError(
                "The value argument must be within the support of the categorical "
                f"distribution (actions in [0, {A}))"
            )
        for key, attr in (("lp", "log_prob"), ("val", "value")):
            parts = [getattr(s, attr) for s in steps]
            if parts[0].dim() == 0:  # (stack needs equal shapes: all 0-d)
                torch.stack(parts, out=host[key])
            else:  # e.g. [1]-shaped
                host[key].copy_(torch.stack(parts).reshape(n))
        host["rew"].numpy()[:] = [s.transition.reward for s in steps]
        host["done"].numpy()[:] = [bool(s.transition.terminated or s.transition.truncated)
                                   for s in steps]

        stage = self._stage.pop(n, None)
        if stage is None:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            stage = views(buf)
            stage["buf"] = buf
            stage["adv"] = torch.empty(n, dtype=torch.float32, device=self.device)
            stage["ret"] = torch.empty(n, dtype=torch.float32, device=self.device)
        self._stage[n] = stage  # most recent last
        while len(self._stage) > 2:
            self._stage.pop(next(iter(self._stage)))
        stage["buf"].copy_(self._host[:nbytes], non_blocking=True)
        if self.device.type == "cuda":
            if self._host_ready is None:
                self._host_ready = torch.cuda.Event()
            self._host_ready.record()
        return stage

    def _update_fused(self, staged: dict, advantages: torch.Tensor,
                      returns: torch.Tensor) -> None:
        """ppo.py:129-171 as VecPPO's fused minibatch loop over the episode's
        arrays: the same torch.randperm draws on the global CPU generator
        (all epochs drawn before the first minibatch, which consumes the
        generator identically: nothing between the reference's draws uses
        it), one upload, two launches per minibatch, one wait-status check.
        An episode as long as the previous one has the same device arrays
        (_upload_rollout), and its loop is replayed from graphs."""
        n = staged["obs"].shape[0]
        if advantages.data_ptr() != staged["adv"].data_ptr():
            staged["adv"].copy_(advantages)
        if returns.data_ptr() != staged["ret"].data_ptr():
            staged["ret"].copy_(returns)
        arrays = (staged["obs"], staged["act"], staged["lp"], staged["adv"], staged["ret"],
                  staged["val"])
        use_graphs = self.graphs and n == self._last_n
        self._last_n = n
        self._vec.update_flat(arrays, self.device, graphs=use_graphs)

    def _update_batch(
        self,
        observations: torch.Tensor,
        actions: torch.Tensor,
        old_log_probs: torch.Tensor,
        advantages: torch.Tensor,
        returns: torch.Tensor,
        old_values: Optional[torch.Tensor] = None,
    ) -> None:
        """ppo.py:141-171.  With the fused update: one fused MLP step over
        the given rows (forward, loss, backward, clip_grad_norm_ and Adam).
        Otherwise: MLP forwards in torch, the fused loss kernel for the loss
        and its gradient, then backward through the MLPs, clip_grad_norm_ and
        Adam.  `old_values` (the rollout's values of the minibatch rows) is
        needed only with PPOConfig.vf_clip, which the reference does not
        have; ValueError if it is missing then."""
        cfg = self.ppo_config
        if cfg.vf_clip is not None and old_values is None:
            raise ValueError("PPOConfig.vf_clip needs the minibatch's old_values")
        if self.fused_update:
            ops.ppo_mlp_cat_step(
                self.policy, self.value, self.optimizer, observations.contiguous(),
                actions.contiguous(), old_log_probs.contiguous(), advantages.contiguous(),
                returns.contiguous(), None if old_values is None else old_values.contiguous(),
                None, cfg.clip_ratio, cfg.vf_clip, cfg.value_coef, cfg.entropy_coef)
            return
        logits = self.policy(observations)
        values = self.value(observations).squeeze(1)
        loss, _ = ops.ppo_loss_discrete(
            logits.contiguous(),
            actions.contiguous(),
            old_log_probs.contiguous(),
            advantages.contiguous(),
            returns.contiguous(),
            values.contiguous(),
            clip_ratio=cfg.clip_ratio,
            vf_clip=cfg.vf_clip,
            value_coef=cfg.value_coef,
            entropy_coef=cfg.entropy_coef,
            old_values=None if old_values is None else old_values.contiguous(),
        )
        self.optimizer.zero_grad()
        loss.backward()
        nn.utils.clip_grad_norm_(self.parameters, cfg.gradient_clip)
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
