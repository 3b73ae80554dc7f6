"""CPU restatement of the reference PPO update path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker or as the timed CPU baseline; the product package
(ppo_amd) never imports it.

Reference: mrhooray/zero-to-hero rl/deep/agents/ppo.py (PPOAgent), whose
update path is pure Python + PyTorch on the CPU.  Every function below cites
the lines it restates.  The loss and gradient arithmetic of the reference
lives in torch (torch.distributions.Categorical, torch.minimum, clamp,
mse_loss, autograd; torch 2.12.0 pinned at rl/uv.lock:842-843, torch 2.10 is
installed here): the loss oracles call those same torch CPU ops, which is the
reference's own call sequence (ppo.py:149-169), and are pinned independently
by finite differences and closed forms in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch
from torch import nn
from torch.distributions import Categorical, Normal

_HERE = os.path.dirname(os.path.abspath(__file__))
_C_LIB = os.path.join(_HERE, "_build", "libgae_ref.so")


# ---------------------------------------------------------------------------
# GAE
# ---------------------------------------------------------------------------
def advantages_python(
    rewards: Sequence[float],
    dones: Sequence[bool],
    values: Sequence[float],
    gamma: float,
    lam: float,
) -> list[float]:
    """Pure-Python restatement of PPOAgent._advantages, ppo.py:173-193.

    One episode; `dones[i]` stands for `terminated or truncated` (:179) and
    `values[i]` for `values[index].item()` (:183, :190).  Returns the Python
    floats before the fp32 cast of :193.  Small inputs only (scalar loop).
    Pinned by the reference's own known answer (test_ppo.py:34-44) and by the
    closed forms and brute-force sum in tests/test_oracle.py.
    """
    advantages = []
    advantage = 0.0
    next_value = 0.0
    for index in reversed(range(len(rewards))):
        mask = 1.0 - float(bool(dones[index]))
        delta = rewards[index] + gamma * next_value * mask - values[index]
        advantage = delta + gamma * lam * mask * advantage
        advantages.append(advantage)
        next_value = values[index]
    advantages.reverse()
    return advantages


def gae_numpy(
    rewards: np.ndarray,
    values: np.ndarray,
    dones: np.ndarray,
    last_value: np.ndarray | None,
    gamma: float,
    lam: float,
) -> tuple[np.ndarray, np.ndarray]:
    """[T,N] generalisation of ppo.py:173-193 (+ returns, :124), numpy fp64.

    Loops over T in reverse, vectorised over the N envs, with the same
    left-to-right operation order as the Python expressions, so each column is
    bit-identical to advantages_python() on that column (numpy float64 ops are
    IEEE binary64, like Python floats).  `last_value` None = zeros (:176).
    Returns (adv fp32, ret fp32) with ret = adv + values in fp32 (:124).
    """
    T, N = rewards.shape
    r = rewards.astype(np.float64)
    v = values.astype(np.float64)
    mask = 1.0 - (dones != 0).astype(np.float64)
    gl = gamma * lam
    adv = np.empty((T, N), dtype=np.float32)
    a = np.zeros(N, dtype=np.float64)
    nv = np.zeros(N) if last_value is None else last_value.astype(np.float64)
    for t in range(T - 1, -1, -1):
        delta = (r[t] + (gamma * nv) * mask[t]) - v[t]
        a = delta + (gl * mask[t]) * a
        adv[t] = a.astype(np.float32)
        nv = v[t]
    ret = adv + values.astype(np.float32)
    return adv, ret


def gae_bruteforce(
    rewards: np.ndarray,
    values: np.ndarray,
    dones: np.ndarray,
    last_value: np.ndarray | None,
    gamma: float,
    lam: float,
) -> np.ndarray:
    """O(T^2) direct sum, an independent statement of the same quantity:

        A_t = sum_{k>=0} (prod_{j<k} gamma*lam*m_{t+j}) * delta_{t+k},
        delta_t = r_t + gamma*m_t*V_{t+1} - V_t,  V_T = last_value,

    with m_t = 1 - done_t.  fp64 (math.fsum per term list); tiny inputs only.
    """
    T, N = rewards.shape
    out = np.zeros((T, N), dtype=np.float64)
    for n in range(N):
        m = [1.0 - float(dones[t, n] != 0) for t in range(T)]
        vnext = [float(values[t + 1, n]) for t in range(T - 1)]
        vnext.append(0.0 if last_value is None else float(last_value[n]))
        deltas = [
            float(rewards[t, n]) + gamma * m[t] * vnext[t] - float(values[t, n])
            for t in range(T)
        ]
        for t in range(T):
            terms = []
            w = 1.0
            for k in range(t, T):
                terms.append(w * deltas[k])
                w *= gamma * lam * m[k]
                if w == 0.0:
                    break
            out[t, n] = math.fsum(terms)
    return out


def build_c() -> str:
    """Compile gae_ref.c with the Makefile beside it; returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _C_LIB


_c_handle = None


def _c_lib():
    global _c_handle
    if _c_handle is None:
        if not os.path.exists(_C_LIB):
            raise RuntimeError(f"{_C_LIB} missing: run oracle.ppo_oracle.build_c()")
        lib = ctypes.CDLL(_C_LIB)
        lib.gae_ref_f64.restype = None
        lib.gae_ref_f64.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int64, ctypes.c_int64, ctypes.c_double, ctypes.c_double,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        _c_handle = lib
    return _c_handle


def gae_c(
    rewards: np.ndarray,
    values: np.ndarray,
    dones: np.ndarray,
    last_value: np.ndarray | None,
    gamma: float,
    lam: float,
) -> tuple[np.ndarray, np.ndarray]:
    """gae_ref.c through ctypes: same contract and bits as gae_numpy(), fast
    enough for the full benchmark shapes (8M-17M elements in well under 1 s)."""
    T, N = rewards.shape
    r = np.ascontiguousarray(rewards, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    d = np.ascontiguousarray(dones != 0, dtype=np.uint8)
    lv = None if last_value is None else np.ascontiguousarray(last_value, dtype=np.float32)
    adv = np.empty((T, N), dtype=np.float32)
    ret = np.empty((T, N), dtype=np.float32)
    _c_lib().gae_ref_f64(
        r.ctypes.data, v.ctypes.data, d.ctypes.data,
        None if lv is None else lv.ctypes.data,
        T, N, float(gamma), float(lam), adv.ctypes.data, ret.ctypes.data,
    )
    return adv, ret


# ---------------------------------------------------------------------------
# Advantage normalisation
# ---------------------------------------------------------------------------
def normalize_reference(advantages: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """ppo.py:126-127 verbatim in torch CPU ops: unbiased std, eps added to
    the std, and no normalisation at all for a single element."""
    if len(advantages) > 1:
        return (advantages - advantages.mean()) / (advantages.std() + eps)
    return advantages


# ---------------------------------------------------------------------------
# Loss forward + backward
# ---------------------------------------------------------------------------
def _value_loss(values, returns, old_values, vf_clip):
    """ppo.py:160 (mse_loss, mean, no 1/2) when vf_clip is None; otherwise the
    clipped form mean(max((v-R)^2, (v_old + clamp(v-v_old, -c, c) - R)^2)),
    which reduces to ppo.py:160 as c -> infinity (no reference code: the
    reference has no value clipping)."""
    if vf_clip is None:
        return nn.functional.mse_loss(values, returns)
    v_clipped = old_values + (values - old_values).clamp(-vf_clip, vf_clip)
    return torch.maximum((values - returns) ** 2, (v_clipped - returns) ** 2).mean()


def _policy_terms(log_probs, old_log_probs, advantages, clip_ratio):
    """ppo.py:154-159."""
    ratio = torch.exp(log_probs - old_log_probs)
    clipped_ratio = ratio.clamp(1.0 - clip_ratio, 1.0 + clip_ratio)
    policy_loss = -torch.minimum(ratio * advantages, clipped_ratio * advantages)
    return ratio, policy_loss


def loss_categorical_reference(
    logits: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: torch.Tensor | None = None,
    clip_ratio: float = 0.2,
    vf_clip: float | None = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> dict:
    """PPOAgent._update_batch loss and backward, ppo.py:150-169, on CPU.

    The logits and values are leaves here (the MLPs of :149/:152 sit outside
    the fused op); returns the scalars and d loss / d logits, d loss / d values
    from torch autograd.  Computes in the dtype of `logits` (fp32 or fp64).
    """
    logits = logits.detach().cpu().clone().requires_grad_(True)
    values = values.detach().cpu().clone().requires_grad_(True)
    dt = logits.dtype
    actions = actions.detach().cpu().long()
    old_log_probs = old_log_probs.detach().cpu().to(dt)
    advantages = advantages.detach().cpu().to(dt)
    returns = returns.detach().cpu().to(dt)
    if old_values is not None:
        old_values = old_values.detach().cpu().to(dt)

    distribution = Categorical(logits=logits)                       # :150
    log_probs = distribution.log_prob(actions)                      # :151
    ratio, policy_loss = _policy_terms(log_probs, old_log_probs, advantages, clip_ratio)
    value_loss = _value_loss(values, returns, old_values, vf_clip)  # :160
    entropy_bonus = distribution.entropy()                          # :161
    loss = (                                                        # :163-167
        policy_loss.mean()
        + value_coef * value_loss
        - entropy_coef * entropy_bonus.mean()
    )
    loss.backward()                                                 # :169
    with torch.no_grad():
        approx_kl = (old_log_probs - log_probs).mean()
        clipfrac = ((ratio - 1.0).abs() > clip_ratio).to(dt).mean()
    return {
        "loss": loss.detach(),
        "policy": policy_loss.mean().detach(),
        "value": value_loss.detach(),
        "entropy": entropy_bonus.mean().detach(),
        "approx_kl": approx_kl,
        "clipfrac": clipfrac,
        "ratio": ratio.detach(),
        "dlogits": logits.grad.detach(),
        "dvalues": values.grad.detach(),
    }


def loss_gaussian_reference(
    mu: torch.Tensor,
    log_std: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: torch.Tensor | None = None,
    clip_ratio: float = 0.2,
    vf_clip: float | None = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> dict:
    """Gaussian-policy variant of loss_categorical_reference (no reference
    code: the reference policy is Categorical only, ppo.py:150).  The policy is
    Normal(mu, exp(log_std)) with a state-independent log_std[D]; log_prob and
    entropy are summed over the action dims; the rest is ppo.py:154-169."""
    mu = mu.detach().cpu().clone().requires_grad_(True)
    log_std = log_std.detach().cpu().clone().requires_grad_(True)
    values = values.detach().cpu().clone().requires_grad_(True)
    dt = mu.dtype
    actions = actions.detach().cpu().to(dt)
    old_log_probs = old_log_probs.detach().cpu().to(dt)
    advantages = advantages.detach().cpu().to(dt)
    returns = returns.detach().cpu().to(dt)
    if old_values is not None:
        old_values = old_values.detach().cpu().to(dt)

    distribution = Normal(mu, log_std.exp())
    log_probs = distribution.log_prob(actions).sum(-1)
    ratio, policy_loss = _policy_terms(log_probs, old_log_probs, advantages, clip_ratio)
    value_loss = _value_loss(values, returns, old_values, vf_clip)
    entropy_bonus = distribution.entropy().sum(-1)
    loss = (
        policy_loss.mean()
        + value_coef * value_loss
        - entropy_coef * entropy_bonus.mean()
    )
    loss.backward()
    with torch.no_grad():
        approx_kl = (old_log_probs - log_probs).mean()
        clipfrac = ((ratio - 1.0).abs() > clip_ratio).to(dt).mean()
    return {
        "loss": loss.detach(),
        "policy": policy_loss.mean().detach(),
        "value": value_loss.detach(),
        "entropy": entropy_bonus.mean().detach(),
        "approx_kl": approx_kl,
        "clipfrac": clipfrac,
        "ratio": ratio.detach(),
        "dmu": mu.grad.detach(),
        "dlog_std": log_std.grad.detach(),
        "dvalues": values.grad.detach(),
    }


# ---------------------------------------------------------------------------
# The whole update, for end-to-end parity of the host driver
# ---------------------------------------------------------------------------


# ---------------------------------------------------------------------------
# Action selection
# ---------------------------------------------------------------------------
def sample_categorical_reference(logits: np.ndarray, uniforms: np.ndarray):
    """Inverse-CDF sampling of Categorical(logits=...) at given uniforms, fp64.

    PPOAgent.select_action (ppo.py:65-79) draws `Categorical(logits).sample()`
    and keeps `.log_prob(action)`; the batched kernel draws the same
    distribution by inverting the CDF at a caller-supplied uniform, which this
    restates: action = min{ j : u < cumsum(softmax(z))_j } (A-1 if none), and
    log_prob = log_softmax(z)[action].  Returns (actions int64 [N], log_probs
    float64 [N], margin [N]) where margin is the distance from u to the
    nearest CDF boundary (rows with a tiny margin may round differently in
    fp32).  Pinned in tests/test_oracle.py by known answers, by the empirical
    frequencies matching softmax, and by the log-probs matching
    torch.distributions.Categorical in fp64.
    """
    z = np.asarray(logits, dtype=np.float64)
    u = np.asarray(uniforms, dtype=np.float64)
    zs = z - z.max(axis=1, keepdims=True)
    p = np.exp(zs)
    p /= p.sum(axis=1, keepdims=True)
    cdf = np.cumsum(p, axis=1)
    actions = (u[:, None] >= cdf).sum(axis=1)
    actions = np.minimum(actions, z.shape[1] - 1)
    logp = zs - np.log(np.exp(zs).sum(axis=1, keepdims=True))
    margin = np.abs(cdf - u[:, None]).min(axis=1)
    return actions, logp[np.arange(z.shape[0]), actions], margin


@dataclass(frozen=True)
class OracleConfig:
    """Defaults of TrainingConfig (rl/deep/type.py:30-41) and PPOConfig
    (ppo.py:15-22) that the update reads."""

    gamma: float = 0.99
    lr: float = 3e-4
    batch_size: int = 128
    epochs: int = 4
    clip_ratio: float = 0.2
    gae_lambda: float = 0.95
    value_coef: float = 0.5
    entropy_coef: float = 0.01
    gradient_clip: float = 0.5


def reference_update(
    policy: nn.Module,
    value: nn.Module,
    optimizer: torch.optim.Optimizer,
    observations: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    old_values: torch.Tensor,
    rewards: Sequence[float],
    dones: Sequence[bool],
    config: OracleConfig = OracleConfig(),
) -> None:
    """PPOAgent._update, ppo.py:113-171, on CPU modules, for one episode.

    Consumes torch's global CPU generator through torch.randperm exactly as
    :130 does, so a caller that seeds it identically sees the same minibatches.
    """
    vals = [float(x) for x in old_values.tolist()]
    adv = torch.as_tensor(
        advantages_python(rewards, dones, vals, config.gamma, config.gae_lambda),
        dtype=torch.float32,
    )                                                               # :123
    returns = adv + old_values                                      # :124
    advantages = normalize_reference(adv)                           # :126-127
    reference_epochs(policy, value, optimizer, observations, actions, old_log_probs,
                     advantages, returns, config)


def reference_epochs(
    policy: nn.Module,
    value: nn.Module,
    optimizer: torch.optim.Optimizer,
    observations: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    config: OracleConfig = OracleConfig(),
    generator: torch.Generator | None = None,
) -> None:
    """The epoch/minibatch loop and _update_batch, ppo.py:129-171, on CPU."""
    params = list(policy.parameters()) + list(value.parameters())
    for _ in range(config.epochs):                                  # :129
        indices = torch.randperm(len(actions), generator=generator)  # :130
        for start in range(0, len(actions), config.batch_size):     # :131
            idx = indices[start : start + config.batch_size]        # :132
            obs_b = observations[idx]
            logits = policy(obs_b)                                  # :149
            distribution = Categorical(logits=logits)
            log_probs = distribution.log_prob(actions[idx])
            values_b = value(obs_b).squeeze(1)                      # :152
            ratio, policy_loss = _policy_terms(
                log_probs, old_log_probs[idx], advantages[idx], config.clip_ratio
            )
            value_loss = nn.functional.mse_loss(values_b, returns[idx])
            entropy_bonus = distribution.entropy()
            loss = (
                policy_loss.mean()
                + config.value_coef * value_loss
                - config.entropy_coef * entropy_bonus.mean()
            )
            optimizer.zero_grad()                                   # :168
            loss.backward()
            nn.utils.clip_grad_norm_(params, config.gradient_clip)  # :170
            optimizer.step()                                        # :171


def update_batch_grads_reference(
    policy: nn.Module,
    value: nn.Module,
    observations: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    old_values: torch.Tensor | None = None,
    clip_ratio: float = 0.2,
    vf_clip: float | None = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> dict:
    """The forward and backward of PPOAgent._update_batch, ppo.py:141-169, on
    CPU modules for one (already gathered) minibatch: the parameter gradients
    of `policy` then `value` (in .parameters() order) and the loss scalars.
    Computes in the modules' dtype; the modules' .grad are left untouched."""
    with torch.enable_grad():
        return _update_batch_grads(policy, value, observations, actions, old_log_probs,
                                   advantages, returns, old_values, clip_ratio, vf_clip,
                                   value_coef, entropy_coef)


def _update_batch_grads(policy, value, observations, actions, old_log_probs, advantages,
                        returns, old_values, clip_ratio, vf_clip, value_coef, entropy_coef):
    params = list(policy.parameters()) + list(value.parameters())
    dt = params[0].dtype
    obs = observations.detach().cpu().to(dt)
    logits = policy(obs)                                            # :149
    values = value(obs).squeeze(1)                                  # :152
    distribution = Categorical(logits=logits)                       # :150
    log_probs = distribution.log_prob(actions.detach().cpu().long())  # :151
    ratio, policy_loss = _policy_terms(log_probs, old_log_probs.detach().cpu().to(dt),
                                       advantages.detach().cpu().to(dt), clip_ratio)
    ov = None if old_values is None else old_values.detach().cpu().to(dt)
    value_loss = _value_loss(values, returns.detach().cpu().to(dt), ov, vf_clip)  # :160
    entropy_bonus = distribution.entropy()                          # :161
    loss = (                                                        # :163-167
        policy_loss.mean()
        + value_coef * value_loss
        - entropy_coef * entropy_bonus.mean()
    )
    grads = torch.autograd.grad(loss, params)                       # :169
    with torch.no_grad():
        approx_kl = (old_log_probs.detach().cpu().to(dt) - log_probs).mean()
        clipfrac = ((ratio - 1.0).abs() > clip_ratio).to(dt).mean()
    return {
        "grads": [g.detach() for g in grads],
        "loss": loss.detach(),
        "policy": policy_loss.mean().detach(),
        "value": value_loss.detach(),
        "entropy": entropy_bonus.mean().detach(),
        "approx_kl": approx_kl,
        "clipfrac": clipfrac,
        "ratio": ratio.detach(),
    }


# ---------------------------------------------------------------------------
# CartPole-v1 dynamics (the reference's environment, rl/deep/cli.py:179-180)
# ---------------------------------------------------------------------------
# The equations are not in the reference's sources: they live in gymnasium
# (>= 1.3 per rl/uv.lock), which is not installed here.  This restates the
# published cart-pole model (Barto, Sutton & Anderson 1983) with gymnasium's
# CartPoleEnv constants and conventions (explicit Euler, tau 0.02, fp64
# state, fp32 observations, |x| > 2.4 or |theta| > 12 degrees terminates,
# reward 1 per step, TimeLimit 500).  Parity with gymnasium itself is
# unpinned; tests/test_oracle.py pins this restatement by an exact rational
# known answer and by mirror symmetry.
CARTPOLE = dict(gravity=9.8, masscart=1.0, masspole=0.1, length=0.5, force_mag=10.0, tau=0.02,
                x_threshold=2.4)


def _cartpole_dynamics(state4, action):
    """One explicit-Euler step of gymnasium's CartPoleEnv (the reference's
    environment, rl/deep/cli.py:179-180) in Python floats: (x, x_dot, theta,
    theta_dot, terminated)."""
    c = CARTPOLE
    total_mass = c["masspole"] + c["masscart"]
    polemass_length = c["masspole"] * c["length"]
    theta_threshold = 12 * 2 * math.pi / 360
    x, x_dot, theta, theta_dot = (float(v) for v in state4)
    force = c["force_mag"] if action == 1 else -c["force_mag"]
    costheta, sintheta = math.cos(theta), math.sin(theta)
    temp = (force + polemass_length * (theta_dot * theta_dot) * sintheta) / total_mass
    thetaacc = (c["gravity"] * sintheta - costheta * temp) / (
        c["length"] * (4.0 / 3.0 - c["masspole"] * (costheta * costheta) / total_mass))
    xacc = temp - polemass_length * thetaacc * costheta / total_mass
    x = x + c["tau"] * x_dot
    x_dot = x_dot + c["tau"] * xacc
    theta = theta + c["tau"] * theta_dot
    theta_dot = theta_dot + c["tau"] * thetaacc
    term = (x < -c["x_threshold"] or x > c["x_threshold"]
            or theta < -theta_threshold or theta > theta_threshold)
    return x, x_dot, theta, theta_dot, term


def cartpole_step_reference(state, actions, steps, reset_uniforms, max_steps=500):
    """One step of N environments in Python floats (fp64), each operation
    rounded on its own: returns (next_state [N,4] f64 after same-step resets,
    obs [N,4] f32, rewards [N] f32, dones [N] u8, terminated [N] u8, steps
    [N] int32)."""
    state = np.asarray(state, np.float64)
    N = state.shape[0]
    nxt = np.empty_like(state)
    dones = np.zeros(N, np.uint8)
    term_out = np.zeros(N, np.uint8)
    steps_out = np.zeros(N, np.int32)
    for n in range(N):
        x, x_dot, theta, theta_dot, term = _cartpole_dynamics(state[n], int(actions[n]))
        t = int(steps[n]) + 1
        done = term or t >= max_steps
        if done:
            u = np.asarray(reset_uniforms[n], np.float64)
            nxt[n] = -0.05 + (0.05 - -0.05) * u
        else:
            nxt[n] = (x, x_dot, theta, theta_dot)
        dones[n], term_out[n], steps_out[n] = done, term, 0 if done else t
    return (nxt, nxt.astype(np.float32), np.ones(N, np.float32), dones, term_out, steps_out)


class CartPoleHost:
    """A single CartPole-v1 environment with gymnasium's API as the runner
    uses it (rl/deep/runner.py:52-84): reset(seed) -> (obs, info), step(a) ->
    (obs, 1.0, terminated, truncated, info), no automatic reset, truncation
    at 500 steps; observation_space.shape == (4,), action_space.n == 2 and
    action_space.seed().  The dynamics are _cartpole_dynamics; the reset state
    is U(-0.05, 0.05)^4 from numpy's default_rng(seed) (gymnasium draws it from
    its own PCG64 stream, which is not reproduced here)."""

    class _Space:
        def __init__(self, shape=None, n=None):
            self.shape, self.n = shape, n

        def seed(self, seed=None):
            return [seed]

    def __init__(self, max_steps: int = 500):
        self.observation_space = self._Space(shape=(4,))
        self.action_space = self._Space(n=2)
        self.max_steps = max_steps
        self.state = np.zeros(4)
        self.steps = 0

    def reset(self, seed=None):
        self.state = np.random.default_rng(seed).uniform(-0.05, 0.05, size=4)
        self.steps = 0
        return self.state.astype(np.float32), {}

    def step(self, action):
        x, x_dot, theta, theta_dot, term = _cartpole_dynamics(self.state, int(action))
        self.state = np.array([x, x_dot, theta, theta_dot])
        self.steps += 1
        trunc = not term and self.steps >= self.max_steps
        return self.state.astype(np.float32), 1.0, bool(term), bool(trunc), {}


def reference_mlp(input_size: int, hidden_size: int, output_size: int) -> nn.Module:
    """MLP of rl/deep/agents/common.py:16-28: Linear-ReLU-Linear-ReLU-Linear,
    constructed in the same order (so one seed gives the same weights)."""
    return nn.Sequential(
        nn.Linear(input_size, hidden_size), nn.ReLU(),
        nn.Linear(hidden_size, hidden_size), nn.ReLU(),
        nn.Linear(hidden_size, output_size),
    )


class ReferenceAgent:
    """PPOAgent of rl/deep/agents/ppo.py:38-171 on the CPU for a CartPole-like
    env: the same seeding (:47), weight construction order, Adam, action
    sampling from a CPU Categorical on the global generator (:65-79), rollout
    bookkeeping (:81-111) and reference_update at the end of an episode."""

    name = "ppo"

    def __init__(self, hidden_size: int = 128, batch_size: int = 128, seed: int = 24,
                 config: OracleConfig | None = None):
        torch.manual_seed(seed)                                          # :47
        self.config = config or OracleConfig(batch_size=batch_size)
        self.policy = reference_mlp(4, hidden_size, 2)                   # :52
        self.value = reference_mlp(4, hidden_size, 1)                    # :53
        self.optimizer = torch.optim.Adam(
            list(self.policy.parameters()) + list(self.value.parameters()), lr=self.config.lr)
        self.rollout, self.pending = [], None

    def start_episode(self, episode: int) -> None:                      # :61-63
        self.rollout, self.pending = [], None

    @torch.no_grad()
    def select_action(self, observation, training: bool = True) -> int:  # :65-79
        obs = torch.as_tensor(observation, dtype=torch.float32)
        logits = self.policy(obs)
        if not training:
            return int(torch.argmax(logits).item())
        dist = Categorical(logits=logits)
        action = dist.sample()
        self.pending = (dist.log_prob(action), self.value(obs).squeeze())
        return int(action.item())

    def update(self, observation, action, reward, next_observation, terminated,
               truncated) -> None:                                       # :81-107
        if self.pending is None:
            return
        self.rollout.append((observation, action, reward, bool(terminated or truncated),
                             self.pending[0], self.pending[1]))
        self.pending = None

    def end_episode(self) -> None:                                       # :109-111
        if not self.rollout:
            return
        obs = torch.as_tensor(np.array([s[0] for s in self.rollout]), dtype=torch.float32)
        actions = torch.as_tensor([s[1] for s in self.rollout], dtype=torch.int64)
        lps = torch.stack([s[4] for s in self.rollout])
        vals = torch.stack([s[5] for s in self.rollout])
        reference_update(self.policy, self.value, self.optimizer, obs, actions, lps, vals,
                         [s[2] for s in self.rollout], [s[3] for s in self.rollout],
                         self.config)


def run_episode(env, agent, episode: int, seed: int, training: bool):
    """rl/deep/runner.py:42-84 (_run_episode): returns (return, length,
    terminated, truncated)."""
    observation, _ = env.reset(seed=seed + episode)
    env.action_space.seed(seed + episode)
    observation = np.asarray(observation, dtype=np.float32)
    agent.start_episode(episode)
    episode_return, length = 0.0, 0
    while True:
        action = agent.select_action(observation, training=training)
        next_observation, reward, terminated, truncated, _ = env.step(action)
        next_observation = np.asarray(next_observation, dtype=np.float32)
        if training:
            agent.update(observation, action, float(reward), next_observation, terminated,
                         truncated)
        episode_return += float(reward)
        length += 1
        observation = next_observation
        if terminated or truncated:
            break
    agent.end_episode()
    return episode_return, length, bool(terminated), bool(truncated)


# ---------------------------------------------------------------------------
# CPU baseline step (bench.py's cpu_baseline leg)
# ---------------------------------------------------------------------------
def cpu_update_step(
    rewards: np.ndarray,
    values: np.ndarray,
    dones: np.ndarray,
    last_value: np.ndarray,
    logits: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    new_values: torch.Tensor,
    old_values: torch.Tensor,
    gamma: float = 0.99,
    lam: float = 0.95,
    clip_ratio: float = 0.2,
    vf_clip: float | None = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> dict:
    """One pass of the hot path on the CPU: GAE (reverse loop over T,
    vectorised over N, ppo.py:173-193 semantics), returns (:124),
    normalisation (:126-127) and the loss forward+backward (:150-169) over all
    T*N samples as one batch, with `new_values` the value head's output and
    `old_values` the rollout values (for value clipping)."""
    adv, ret = gae_numpy(rewards, values, dones, last_value, gamma, lam)
    adv_t = torch.from_numpy(adv).reshape(-1)
    ret_t = torch.from_numpy(ret).reshape(-1)
    adv_n = normalize_reference(adv_t)
    return loss_categorical_reference(
        logits, actions, old_log_probs, adv_n, ret_t, new_values, old_values,
        clip_ratio, vf_clip, value_coef, entropy_coef,
    )
