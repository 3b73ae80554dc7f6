"""End-to-end parity of the host driver: PPOAgent._update and VecPPO.update
(GAE, normalisation and fused loss on the GPU; MLPs, clip_grad_norm_ and Adam
in torch on the GPU) against the CPU restatement of ppo.py:113-171 starting
from identical weights and the identical torch.randperm stream.

Tolerance: parameters after the update agree to 2e-5 absolute (lr = 3e-4;
the residue is fp32 GEMM and reduction-order noise amplified by Adam).
"""

import copy
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import ppo_amd
from oracle import ppo_oracle as ref
from ppo_amd.agent import MLP, PPOAgent, PPOConfig, RolloutStep, TrainingConfig, Transition

pytestmark = pytest.mark.gpu


def cartpole_like():
    return SimpleNamespace(observation_space=SimpleNamespace(shape=(4,)),
                           action_space=SimpleNamespace(n=2))


def _rollout_step(reward, terminated, obs=None, action=0, log_prob=0.0, value=0.0):
    obs = np.zeros(4, dtype=np.float32) if obs is None else obs
    return RolloutStep(
        transition=Transition(observation=obs, action=action, reward=reward,
                              next_observation=obs, terminated=terminated, truncated=False),
        log_prob=torch.as_tensor(log_prob),
        value=torch.as_tensor(value),
    )


def test_ppo_advantages_use_next_step_value(dev):
    """rl/deep/tests/test_ppo.py:34-44, verbatim in intent, on the GPU."""
    config = TrainingConfig(gamma=0.8, hidden_size=16)
    agent = PPOAgent(cartpole_like(), config, PPOConfig(gae_lambda=0.5), device=dev)
    agent.rollout = [_rollout_step(1.0, False), _rollout_step(3.0, True)]
    advantages = agent._advantages(torch.as_tensor([0.5, 1.0]))
    assert advantages.tolist() == pytest.approx([2.1, 2.0])


@pytest.mark.parametrize("T,activation", [(37, "relu"), (200, "tanh")])
def test_agent_update_matches_reference(dev, T, activation):
    config = TrainingConfig(hidden_size=64, batch_size=32)
    agent = PPOAgent(cartpole_like(), config, device=dev, activation=activation)
    torch.manual_seed(config.seed)
    policy = MLP(4, config.hidden_size, 2, activation)
    value = MLP(4, config.hidden_size, 1, activation)
    for a, b in zip(agent.parameters, list(policy.parameters()) + list(value.parameters())):
        assert torch.equal(a.detach().cpu(), b.detach())
    opt = torch.optim.Adam(list(policy.parameters()) + list(value.parameters()), lr=config.lr)

    g = torch.Generator().manual_seed(T)
    obs = (torch.rand(T, 4, generator=g) - 0.5) * 0.1
    with torch.no_grad():
        logits = policy(obs)
        actions = torch.multinomial(torch.softmax(logits, -1), 1, generator=g).squeeze(1)
        lps = torch.log_softmax(logits, -1).gather(1, actions[:, None]).squeeze(1)
        vals = value(obs).squeeze(1)
    dones = [False] * (T - 1) + [True]
    agent.rollout = [
        _rollout_step(1.0, dones[t], obs[t].numpy(), int(actions[t]), lps[t].item(),
                      vals[t].item())
        for t in range(T)
    ]
    torch.manual_seed(1234)
    agent._update()
    torch.manual_seed(1234)
    ref.reference_update(policy, value, opt, obs, actions, lps, vals, [1.0] * T, dones,
                         ref.OracleConfig(batch_size=config.batch_size))
    for a, b in zip(agent.parameters, list(policy.parameters()) + list(value.parameters())):
        torch.testing.assert_close(a.detach().cpu(), b.detach(), rtol=0, atol=2e-5)


def test_vec_update_matches_reference(dev):
    """VecPPO over a [T,N] buffer: GAE with bootstrap + normalisation + the
    minibatch loop, against oracle.gae_numpy + normalize_reference +
    reference_epochs on CPU copies of the same modules."""
    T, N, H = 32, 8, 64
    torch.manual_seed(24)
    policy = MLP(4, H, 2, "tanh")
    value = MLP(4, H, 1, "tanh")
    cpu_policy, cpu_value = copy.deepcopy(policy), copy.deepcopy(value)
    cpu_opt = torch.optim.Adam(list(cpu_policy.parameters()) + list(cpu_value.parameters()),
                               lr=3e-4)
    cfg = PPOConfig()
    vec = ppo_amd.VecPPO(policy.to(dev), value.to(dev), cfg, gamma=0.99, lr=3e-4,
                         batch_size=64, generator=torch.Generator().manual_seed(7))

    g = torch.Generator().manual_seed(5)
    obs = (torch.rand(T, N, 4, generator=g) - 0.5) * 0.1
    with torch.no_grad():
        logits = cpu_policy(obs)
        acts = torch.multinomial(torch.softmax(logits.reshape(-1, 2), -1), 1,
                                 generator=g).reshape(T, N)
        lps = torch.log_softmax(logits, -1).gather(2, acts[..., None]).squeeze(2)
        vals = cpu_value(obs).squeeze(2)
    rewards = torch.ones(T, N)
    dones = (torch.rand(T, N, generator=g) < 1 / 200).to(torch.uint8)
    last_v = torch.randn(N, generator=g)

    buf = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    for t in range(T):
        buf.add(obs[t].to(dev), acts[t].to(torch.int32).to(dev), rewards[t].to(dev),
                dones[t].to(dev), vals[t].to(dev), lps[t].to(dev))
    buf.finish(last_v.to(dev))
    vec.update(buf)

    adv, ret = ref.gae_numpy(rewards.numpy(), vals.numpy(), dones.numpy(), last_v.numpy(),
                             0.99, 0.95)
    adv_n = ref.normalize_reference(torch.from_numpy(adv).reshape(-1))
    ref.reference_epochs(cpu_policy, cpu_value, cpu_opt, obs.reshape(-1, 4), acts.reshape(-1),
                         lps.reshape(-1), adv_n, torch.from_numpy(ret).reshape(-1),
                         ref.OracleConfig(batch_size=64),
                         generator=torch.Generator().manual_seed(7))
    for a, b in zip(vec.parameters, list(cpu_policy.parameters()) + list(cpu_value.parameters())):
        torch.testing.assert_close(a.detach().cpu(), b.detach(), rtol=0, atol=2e-5)
