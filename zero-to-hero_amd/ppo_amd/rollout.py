"""Env-contiguous [T,N] rollout buffer and the vectorised PPO update.

The reference stores one episode as a Python list of RolloutStep records and
stacks them at update time (rl/deep/agents/ppo.py:93-106, :114-122).  Here the
rollout of N parallel environments lives on the device as dense [T,N] arrays,
row t holding step t of every env (element (t, n) at t*N + n): exactly the
layout the GAE kernel streams.  `VecPPO.update` is PPOAgent._update
(ppo.py:113-139) over the flattened T*N samples.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import ops
from .agent import PPOConfig
from .optim import ClippedAdam


class RolloutBuffer:
    """Device-resident [T,N] rollout storage.

    Fields: observations [T,N,*obs_shape] f32, actions [T,N] int32 (discrete)
    or [T,N,D] f32 (continuous), rewards/values/log_probs [T,N] f32,
    dones [T,N] uint8 (terminated or truncated), last_value [N] f32 (the value
    of the state after step T-1, used to bootstrap).
    """

    def __init__(
        self,
        T: int,
        N: int,
        obs_shape: tuple,
        device: str | torch.device = "cuda",
        action_dim: Optional[int] = None,
    ) -> None:
        if T <= 0 or N <= 0:
            raise ValueError(f"T and N must be positive, got T={T}, N={N}")
        dev = torch.device(device)
        self.T, self.N, self.device = T, N, dev
        f32 = dict(dtype=torch.float32, device=dev)
        self.observations = torch.zeros((T, N, *obs_shape), **f32)
        if action_dim is None:
            self.actions = torch.zeros((T, N), dtype=torch.int32, device=dev)
        else:
            self.actions = torch.zeros((T, N, action_dim), **f32)
        self.rewards = torch.zeros((T, N), **f32)
        self.values = torch.zeros((T, N), **f32)
        self.log_probs = torch.zeros((T, N), **f32)
        self.dones = torch.zeros((T, N), dtype=torch.uint8, device=dev)
        self.last_value = torch.zeros(N, **f32)
        self.step = 0
        self._gae_out: Optional[list] = None  # normalised advantages, returns ([T,N] each)

    def add(self, observations, actions, rewards, dones, values, log_probs) -> None:
        """Store step `self.step` for all N envs (ppo.py:93-106, batched)."""
        if self.step >= self.T:
            raise IndexError(f"rollout buffer is full (T={self.T})")
        t = self.step
        self.observations[t].copy_(observations)
        self.actions[t].copy_(actions)
        self.rewards[t].copy_(rewards)
        self.dones[t].copy_(dones)
        self.values[t].copy_(values)
        self.log_probs[t].copy_(log_probs)
        self.step += 1

    def add_outcome(self, rewards, dones) -> None:
        """Complete step `self.step` after VecPPO.act(obs, buffer=self) has
        written its observations, actions, log-probs and values: store the
        environment's rewards and dones and advance."""
        if self.step >= self.T:
            raise IndexError(f"rollout buffer is full (T={self.T})")
        self.rewards[self.step].copy_(rewards)
        self.dones[self.step].copy_(dones)
        self.step += 1

    def finish(self, last_value: Optional[torch.Tensor] = None) -> None:
        """Set the bootstrap values (None: zeros, the reference's episode end)."""
        if last_value is None:
            self.last_value.zero_()
        else:
            self.last_value.copy_(last_value)

    def reset(self) -> None:
        self.step = 0

    def compute_advantages(self, gamma: float = 0.99, lam: float = 0.95,
                           normalize: bool = True, eps: float = 1e-8):
        """(advantages, returns, normalized advantages) over the filled steps,
        all [T,N] fp32 (ppo.py:123-127 generalised).  Without `normalize` the
        third item is None."""
        T = self.step
        r, v, d = self.rewards[:T], self.values[:T], self.dones[:T]
        if normalize:
            return ops.gae_normalize(r, v, d, self.last_value, gamma, lam, eps)
        adv, ret = ops.gae(r, v, d, self.last_value, gamma, lam)
        return adv, ret, None

    def _advantages_in_place(self, gamma: float, lam: float, eps: float = 1e-8):
        """compute_advantages(normalize=True) into storage the buffer keeps:
        the same addresses on every call (graph replays read them), contents
        overwritten by the next call.  The raw advantages are not kept (the
        first and third items are the normalised ones)."""
        T = self.step
        if self._gae_out is None:
            self._gae_out = [torch.empty((self.T, self.N), dtype=torch.float32, device=self.device)
                             for _ in range(2)]
        out = tuple(o[:T] for o in self._gae_out)
        r, v, d = self.rewards[:T], self.values[:T], self.dones[:T]
        return ops.gae_normalize(r, v, d, self.last_value, gamma, lam, eps, out=out,
                                 keep_raw=False)


class VecPPO:
    """PPOAgent._update (ppo.py:113-171) for a [T,N] rollout.

    `policy` maps observations to logits [B,A] (categorical) or to mu [B,D]
    (gaussian, with the state-independent `log_std` parameter); `value` maps
    observations to [B,1].  Minibatches come from torch.randperm on the CPU
    generator `generator` (default: the global one, as ppo.py:130 uses).
    With `fused_update` (default), the minibatch gather is one ppo_gather_rows
    launch and clip_grad_norm_ + Adam is ClippedAdam (two launches); otherwise
    torch indexing, clip_grad_norm_ and torch.optim.Adam are used.

    With `fused_mlp` (default: whenever `fused_update` is on, the policy is
    categorical and both networks are MLPs that ops.mlp_fusable accepts) each
    minibatch's gather, MLP forwards, loss and backward are the two launches
    of ops.ppo_mlp_cat_grads, which write the parameters' gradients directly,
    and the clip + Adam step joins the second (ops.ppo_mlp_cat_step: two
    launches per minibatch, three when the reduction's grid cannot be
    resident at once).

    With `graphs=True` (requires `fused_update`) the minibatch loop is replayed
    from CUDA/HIP graphs: the whole update runs on a private stream; the
    graphs read the rollout buffer's own storage (its arrays and the advantage
    outputs it keeps) and one [epochs, n] device tensor of permutations, which
    is the only copy per update.  The first update of a buffer runs its first
    epoch eagerly (the warm-up that initialises library handles and autograd
    state), then captures every epoch's minibatch sequence as graphs of
    `graph_chunk` minibatches and replays them; later updates of the same
    buffer only replay.  Graphs are kept for the two most recent buffers.
    The results equal the eager fused path's: the same kernels run on the
    same data.

    `check_waits` reports in-kernel waits that gave up (GAE resident pass,
    the losses' in-kernel finish, fused clip + Adam) as PPOLibraryError
    (PPO_ERR_WAIT_TIMEOUT): "deferred" (default, also True) checks each
    update's status at the end of the next update (ops.WaitPoller: no
    synchronisation per update) and `flush_waits()` checks at once; "sync"
    synchronises at the end of every update (ops.check_waits); False does
    not check.
    """

    def __init__(
        self,
        policy: nn.Module,
        value: nn.Module,
        ppo_config: PPOConfig = PPOConfig(),
        gamma: float = 0.99,
        lr: float = 3e-4,
        batch_size: int = 128,
        log_std: Optional[nn.Parameter] = None,
        generator: Optional[torch.Generator] = None,
        fused_update: bool = True,
        graphs: bool = False,
        graph_chunk: int = 64,
        fused_mlp: Optional[bool] = None,
        check_waits: bool | str = "deferred",
    ) -> None:
        self.policy, self.value = policy, value
        if check_waits not in (True, False, "deferred", "sync"):
            raise ValueError(f"check_waits must be True, False, 'deferred' or 'sync', got "
                             f"{check_waits!r}")
        self.check_waits = check_waits
        self._poller = ops.WaitPoller()
        self.ppo_config, self.gamma, self.batch_size = ppo_config, gamma, batch_size
        self.log_std = log_std
        self.generator = generator
        self.parameters = list(policy.parameters()) + list(value.parameters())
        if log_std is not None:
            self.parameters.append(log_std)
        self.fused = fused_update
        if graphs and not fused_update:
            raise ValueError("graphs=True needs fused_update=True")
        if graph_chunk < 1:
            raise ValueError(f"graph_chunk must be >= 1, got {graph_chunk}")
        self.graphs, self.graph_chunk = graphs, graph_chunk
        self._plans: dict = {}  # (shape, storage) key -> _GraphPlan, two at most
        self._collect_plans: dict = {}  # (env, buffer, shapes) -> _CollectPlan, two at most
        self._rollout_u: Optional[torch.Tensor] = None  # uniforms of the fused rollout
        self._plan: Optional[_GraphPlan] = None  # the most recently used
        self._side_stream: Optional[torch.cuda.Stream] = None
        self._perms = _PermUploader()
        can_fuse = fused_update and log_std is None and ops.mlp_fusable(policy, value)
        if fused_mlp and not can_fuse:
            raise ValueError("fused_mlp needs fused_update, a categorical policy and MLPs that "
                             "ops.mlp_fusable accepts")
        self.fused_mlp = can_fuse if fused_mlp is None else bool(fused_mlp)
        self._scalars: Optional[torch.Tensor] = None
        if self.fused_mlp:
            # gradients exist before any graph capture; the kernel overwrites them
            for p in self.parameters:
                if p.grad is None:
                    p.grad = torch.zeros_like(p)
            self._scalars = torch.zeros(6, dtype=torch.float32, device=self.parameters[0].device)
        if fused_update:
            self.optimizer = ClippedAdam(self.parameters, lr=lr,
                                         max_grad_norm=ppo_config.gradient_clip,
                                         capturable=graphs)
            # the fused MLP step and captured graphs write into the gradient buffers
            self.optimizer.keep_grads = self.fused_mlp or graphs
        else:
            self.optimizer = torch.optim.Adam(self.parameters, lr=lr)

    @torch.no_grad()
    def act(self, observations: torch.Tensor, buffer: Optional[RolloutBuffer] = None,
            generator: Optional[torch.Generator] = None,
            uniforms: Optional[torch.Tensor] = None):
        """PPOAgent.select_action (ppo.py:65-79) for all N envs at once.

        Runs the policy and value networks on observations [N, *obs_shape],
        then one sampling launch draws every env's action (from uniforms /
        normals drawn on the device with `generator`) and its log-prob.  With
        `buffer`, the observations, actions, log-probs and values are written
        straight into row `buffer.step` (complete it with
        buffer.add_outcome(rewards, dones)).  Returns (actions, log_probs,
        values), views of that row when a buffer is given.
        """
        if self.fused_mlp and observations.dim() == 2:
            outs: dict = {}
            if buffer is not None:
                if buffer.step >= buffer.T:
                    raise IndexError(f"rollout buffer is full (T={buffer.T})")
                t = buffer.step
                outs = dict(observations_out=buffer.observations[t],
                            actions_out=buffer.actions[t], log_probs_out=buffer.log_probs[t],
                            values_out=buffer.values[t])
            return ops.mlp_act_categorical(self.policy, self.value, observations.contiguous(),
                                           uniforms=uniforms, generator=generator, **outs)
        values = self.value(observations).reshape(-1).contiguous()
        if buffer is not None:
            if buffer.step >= buffer.T:
                raise IndexError(f"rollout buffer is full (T={buffer.T})")
            t = buffer.step
            buffer.observations[t].copy_(observations)
            outs = dict(actions_out=buffer.actions[t], log_probs_out=buffer.log_probs[t],
                        values_out=buffer.values[t])
        else:
            outs = dict(values_out=torch.empty_like(values))
        if self.log_std is None:
            logits = self.policy(observations).contiguous()
            acts, logp = ops.sample_categorical(logits, generator=generator, values=values,
                                                **outs)
        else:
            mu = self.policy(observations).contiguous()
            acts, logp = ops.sample_gaussian(mu, self.log_std.detach(), generator=generator,
                                             values=values, **outs)
        return acts, logp, outs["values_out"]

    @torch.no_grad()
    def collect(self, env, buffer: RolloutBuffer, observations: torch.Tensor,
                generator: Optional[torch.Generator] = None, bootstrap: bool = True,
                graphs: Optional[bool] = None, fused: Optional[bool] = None):
        """Fill `buffer` with buffer.T steps of the vectorised environment
        `env` (an object with step(actions int32 [N]) -> (observations,
        rewards, dones, ...), e.g. CartPoleVec), starting from
        `observations` [N, *obs_shape]: the rollout loop of
        rl/deep/runner.py:56-74 for N environments, with select_action
        (ppo.py:65-79) batched by act().  With `bootstrap` the value of the
        state after the last step seeds the advantages of environments still
        running (masked for those whose episode just ended); without it the
        reference's zero is used.  Returns the observations after the last
        step (a copy).

        With `graphs` (default: the VecPPO's `graphs` setting) and an
        environment with step_into(..., reset_uniforms) and the fused MLP
        path, the T steps are replayed from one HIP graph: the rollout's
        random numbers (action uniforms [T,N], reset uniforms [T,N,4]) are
        drawn in one launch first and read by the graph; the first call for
        a (environment, buffer) pair runs eagerly and captures.

        With `fused` (default: whenever possible) a CartPoleVec environment
        and 4-H-H-2 / 4-H-H-1 MLPs on the fused path, the whole rollout is
        one launch (ops.mlp_cartpole_rollout) on uniforms drawn the same way,
        so it fills the buffer exactly as the per-step path does."""
        if fused is not False and self._cartpole_fusable(env, observations):
            return self._collect_fused(env, buffer, observations, generator, bootstrap)
        if fused:
            raise ValueError("fused collection needs a CartPoleVec, the fused MLP path and "
                             "4-H-H-2 / 4-H-H-1 networks")
        use_graph = self.graphs if graphs is None else graphs
        if (use_graph and self.fused_mlp and hasattr(env, "step_into")
                and observations.dim() == 2):
            return self._collect_graphed(env, buffer, observations, generator, bootstrap)
        buffer.reset()
        obs = observations
        into = hasattr(env, "step_into")
        for _ in range(buffer.T):
            t = buffer.step
            acts, _, _ = self.act(obs, buffer=buffer, generator=generator)
            if into:  # the environment writes the buffer row itself
                obs = env.step_into(acts, buffer.rewards[t], buffer.dones[t])
                buffer.step += 1
            else:
                obs, rewards, dones = env.step(acts)[:3]
                buffer.add_outcome(rewards, dones)
        obs = obs.clone()
        buffer.finish(self.value(obs).reshape(-1) if bootstrap else None)
        return obs

    def _cartpole_fusable(self, env, observations) -> bool:
        from .env import CartPoleVec
        if not (self.fused_mlp and isinstance(env, CartPoleVec) and observations.dim() == 2):
            return False
        lp, _ = ops.mlp_structure(self.policy)
        return lp[0].in_features == 4 and lp[2].out_features == 2

    def _collect_fused(self, env, buffer, observations, generator, bootstrap):
        T, N, dev = buffer.T, buffer.N, buffer.device
        u = self._rollout_u
        if u is None or tuple(u.shape) != (T, 5 * N) or u.device != dev:
            u = self._rollout_u = torch.empty((T, 5 * N), dtype=torch.float32, device=dev)
        # the layout of the graphed path's draw (_CollectPlan), so both paths
        # consume the same numbers
        torch.rand(u.shape, generator=generator, device=dev, out=u)
        buffer.reset()
        ops.mlp_cartpole_rollout(self.policy, self.value, env, buffer, observations.contiguous(),
                                 u[:, :N], u[:, N:].view(T, N, 4))
        buffer.step = T
        obs = env.obs.clone()
        buffer.finish(self.value(obs).reshape(-1) if bootstrap else None)
        return obs

    def _collect_graphed(self, env, buffer, observations, generator, bootstrap):
        # The plan keeps the environment and the buffer alive, so their ids
        # (and the storage its graph reads and writes) cannot be reused while
        # the plan exists; at most two plans are kept, most recent last.
        key = (id(env), id(buffer), buffer.T, buffer.N, tuple(observations.shape))
        plan = self._collect_plans.pop(key, None)
        dev = buffer.device
        if plan is None or plan.env is not env or plan.buffer is not buffer:
            plan = _CollectPlan(env, buffer, observations, dev)
        self._collect_plans[key] = plan
        while len(self._collect_plans) > 2:
            self._collect_plans.pop(next(iter(self._collect_plans)))
        torch.rand(plan.u.shape, generator=generator, device=dev, out=plan.u)
        plan.obs0.copy_(observations)
        if plan.graph is None and plan.warm:
            if self._side_stream is None:
                self._side_stream = torch.cuda.Stream(device=dev)
            s = self._side_stream
            s.wait_stream(torch.cuda.current_stream(dev))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._collect_steps(env, buffer, plan)
            torch.cuda.current_stream(dev).wait_stream(s)
            plan.graph = g
        if plan.graph is not None:
            plan.graph.replay()
        else:
            self._collect_steps(env, buffer, plan)  # warm-up, eager
            plan.warm = True
        buffer.step = buffer.T
        obs = env.obs.clone()
        buffer.finish(self.value(obs).reshape(-1) if bootstrap else None)
        return obs

    def _collect_steps(self, env, buffer, plan) -> None:
        buffer.reset()
        obs = plan.obs0
        for t in range(buffer.T):
            acts, _, _ = self.act(obs, buffer=buffer, uniforms=plan.uact[t])
            obs = env.step_into(acts, buffer.rewards[t], buffer.dones[t],
                                reset_uniforms=plan.ureset[t])
            buffer.step += 1

    def update(self, buffer: RolloutBuffer) -> dict:
        """Run `epochs` passes of shuffled minibatches; returns the last
        minibatch's loss scalars (device tensors)."""
        cfg = self.ppo_config
        adv, ret, adv_n = buffer._advantages_in_place(self.gamma, cfg.gae_lambda)
        T = buffer.step
        n = T * buffer.N
        if n <= 1:
            adv_n = adv
        obs = buffer.observations[:T].reshape(n, *buffer.observations.shape[2:]).contiguous()
        acts = buffer.actions[:T].reshape(n, *buffer.actions.shape[2:]).contiguous()
        old_lp = buffer.log_probs[:T].reshape(n).contiguous()
        old_v = buffer.values[:T].reshape(n).contiguous()
        adv_f, ret_f = adv_n.reshape(n).contiguous(), ret.reshape(n).contiguous()
        return self.update_flat((obs, acts, old_lp, adv_f, ret_f, old_v), buffer.device)

    def update_flat(self, arrays: tuple, device: torch.device,
                    graphs: Optional[bool] = None) -> dict:
        """The epoch/minibatch loop (ppo.py:129-171) over flattened rollout
        arrays (observations [n,...], actions [n(,D)], old_log_probs,
        advantages (normalised), returns, old_values [n]): `epochs`
        permutations from torch.randperm on `generator`, drawn together on
        the host and uploaded in one copy, sliced into minibatches on the
        device.  `graphs` overrides the constructor's choice for this call;
        graph plans are keyed on the arrays' storage, so repeated calls replay
        only when the same tensors are passed again."""
        use_graphs = self.graphs if graphs is None else graphs
        if use_graphs and not self.fused:
            raise ValueError("graphs need fused_update=True")
        if use_graphs:
            stats = self._update_graphed(device, arrays)
        else:
            cfg = self.ppo_config
            n = arrays[0].shape[0]
            perms = self._perms.upload(n, cfg.epochs, self.generator, arrays[0].device)
            stats = {}
            for e in range(cfg.epochs):
                for start in range(0, n, self.batch_size):
                    stats = self._minibatch(perms[e, start : start + self.batch_size], arrays)
        if self.check_waits == "sync":
            ops.check_waits(device)
        elif self.check_waits:
            self._poller.check(arrays[0].device)
        return stats

    def flush_waits(self) -> None:
        """Reports at once (synchronising) any in-kernel wait that gave up in
        the updates not yet checked."""
        self._poller.flush(self.parameters[0].device)

    def _minibatch(self, idx: torch.Tensor, arrays: tuple) -> dict:
        """One minibatch (rows idx of the flattened rollout arrays): forward,
        loss, backward and optimizer step."""
        if self.fused_mlp and arrays[0].dim() == 2:
            cfg = self.ppo_config
            obs, acts, old_lp, adv, ret, old_v = arrays
            # gradients, clip to cfg.gradient_clip and Adam: two launches
            stats, _ = ops.ppo_mlp_cat_step(
                self.policy, self.value, self.optimizer, obs, acts, old_lp, adv, ret,
                old_v if cfg.vf_clip is not None else None, idx, cfg.clip_ratio, cfg.vf_clip,
                cfg.value_coef, cfg.entropy_coef, scalars_out=self._scalars)
            return stats
        if self.fused:
            batch = ops.gather_rows(idx, *arrays)
        else:
            batch = [x[idx] for x in arrays]
        return self._update_batch(*batch)

    def update_graphed_ready(self) -> bool:
        """True once graphs are captured for the current rollout shape."""
        return self._plan is not None and bool(self._plan.graphs)

    def _update_graphed(self, device: torch.device, arrays: tuple) -> dict:
        cfg = self.ppo_config
        n, B = arrays[0].shape[0], self.batch_size
        key = (n, B, cfg.epochs) + tuple(
            (a.dtype, tuple(a.shape[1:]), a.data_ptr()) for a in arrays)
        if self._side_stream is None:
            self._side_stream = torch.cuda.Stream(device=device)
        s = self._side_stream
        caller = torch.cuda.current_stream(device)
        s.wait_stream(caller)
        with torch.cuda.stream(s):
            plan = self._plans.pop(key, None)
            if plan is None:
                plan = _GraphPlan(key, arrays, n, B, cfg.epochs, device)
            self._plans[key] = plan  # most recent last
            while len(self._plans) > 2:
                self._plans.pop(next(iter(self._plans)))
            self._plan = plan
            # this update's permutations: written on the host into one of two
            # pinned buffers (the other may still be read by the previous
            # update's upload), then uploaded by a kernel launch
            k = plan.flip
            plan.flip ^= 1
            if plan.host_events[k] is not None:
                plan.host_events[k].synchronize()
            host = plan.perms_host[k]
            for e in range(cfg.epochs):
                torch.randperm(n, generator=self.generator, out=host[e])
            ops.copy_pinned_to_device(plan.perms, host)
            ev = torch.cuda.Event()
            ev.record(s)
            plan.host_events[k] = ev
            first = 0
            if not plan.graphs:
                for j in range(plan.nmb):
                    self._graph_minibatch(plan, 0, j)
                self._capture(plan, s)
                first = 1
            for e in range(first, cfg.epochs):
                for g in plan.graphs[e]:
                    g.replay()
            stats = plan.stats
        caller.wait_stream(s)
        return stats

    def _graph_minibatch(self, plan: "_GraphPlan", e: int, j: int) -> dict:
        idx = plan.perms[e, j * plan.B : (j + 1) * plan.B]
        return self._minibatch(idx, plan.arrays)

    def _capture(self, plan: "_GraphPlan", stream: torch.cuda.Stream) -> None:
        pool = torch.cuda.graph_pool_handle()
        refs: list = []
        ops._WORKSPACES.capture_refs = refs
        try:
            stats: dict = {}
            for e in range(plan.epochs):
                seq = []
                for c in range(0, plan.nmb, self.graph_chunk):
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, pool=pool, stream=stream):
                        for j in range(c, min(c + self.graph_chunk, plan.nmb)):
                            stats = self._graph_minibatch(plan, e, j)
                    seq.append(g)
                plan.graphs.append(seq)
        except BaseException:
            plan.graphs.clear()
            raise
        finally:
            ops._WORKSPACES.capture_refs = None
        plan.stats, plan.refs = stats, refs

    def _update_batch(self, observations, actions, old_log_probs, advantages, returns,
                      old_values) -> dict:
        cfg = self.ppo_config
        values = self.value(observations).squeeze(1).contiguous()
        if self.log_std is None:
            logits = self.policy(observations).contiguous()
            loss, stats = ops.ppo_loss_discrete(
                logits, actions.contiguous(), old_log_probs, advantages, returns, values,
                old_values if cfg.vf_clip is not None else None,
                cfg.clip_ratio, cfg.vf_clip, cfg.value_coef, cfg.entropy_coef,
            )
        else:
            mu = self.policy(observations).contiguous()
            loss, stats = ops.ppo_loss_gaussian(
                mu, self.log_std, actions.contiguous(), old_log_probs, advantages, returns,
                values, old_values if cfg.vf_clip is not None else None,
                cfg.clip_ratio, cfg.vf_clip, cfg.value_coef, cfg.entropy_coef,
            )
        self.optimizer.zero_grad()
        loss.backward()
        if self.fused:
            self.optimizer.step()  # clips to cfg.gradient_clip, then Adam
        else:
            nn.utils.clip_grad_norm_(self.parameters, cfg.gradient_clip)
            self.optimizer.step()
        return stats


class _PermUploader:
    """The eager loop's permutations: `epochs` rows of torch.randperm(n) drawn
    on the host into one of two pinned buffers (the other may still be read
    by the previous upload) and copied to one device buffer in one launch.
    The device buffer is reused: the next upload is ordered after the
    previous update's kernels on the same stream."""

    def __init__(self) -> None:
        self.host: list = [None, None]
        self.events: list = [None, None]
        self.dev: Optional[torch.Tensor] = None
        self.flip = 0

    def upload(self, n: int, epochs: int, generator, device) -> torch.Tensor:
        k = self.flip
        self.flip ^= 1
        if self.events[k] is not None:
            self.events[k].synchronize()
        need = epochs * n
        if self.host[k] is None or self.host[k].numel() < need:
            self.host[k] = torch.empty(max(need, 1024), dtype=torch.int64, pin_memory=True)
        if self.dev is None or self.dev.numel() < need or self.dev.device != device:
            self.dev = torch.empty(max(need, 1024), dtype=torch.int64, device=device)
        host = self.host[k][:need].view(epochs, n)
        for e in range(epochs):
            torch.randperm(n, generator=generator, out=host[e])
        dev = self.dev[:need].view(epochs, n)
        ops.copy_pinned_to_device(dev, host)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        self.events[k] = ev
        return dev


class _GraphPlan:
    """Captured graphs of VecPPO's minibatch loop for one rollout: `arrays`
    are the flattened rollout arrays the graphs read (held, so their storage
    stays allocated while the graphs exist), `perms` the update's [epochs, n]
    permutations (row e's slices are epoch e's minibatch indices), `graphs`
    one list of graphs per epoch."""

    def __init__(self, key, arrays, n: int, B: int, epochs: int, device) -> None:
        self.key, self.n, self.B, self.epochs = key, n, B, epochs
        self.nmb = (n + B - 1) // B
        self.arrays = tuple(arrays)
        self.perms = torch.empty((epochs, n), dtype=torch.int64, device=device)
        self.perms_host = [torch.empty((epochs, n), dtype=torch.int64, pin_memory=True)
                           for _ in range(2)]
        self.host_events: list = [None, None]
        self.flip = 0
        self.graphs: list = []
        self.stats: dict = {}
        self.refs: list = []


class _CollectPlan:
    """Static inputs of a captured collection loop: the starting observations
    and the rollout's uniforms, one [T, 5N] draw: per step N action uniforms,
    then N x 4 reset uniforms (each step's slices contiguous)."""

    def __init__(self, env, buffer, observations: torch.Tensor, device) -> None:
        T, N = buffer.T, buffer.N
        self.env, self.buffer = env, buffer
        self.obs0 = torch.empty_like(observations)
        self.u = torch.empty((T, 5 * N), dtype=torch.float32, device=device)
        self.uact = self.u[:, :N]
        self.ureset = self.u[:, N:].view(T, N, 4)
        self.graph = None
        self.warm = False
