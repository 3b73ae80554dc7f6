"""The method patches of ppo_amd.reference_patch applied to a class shaped
like the reference's PPOAgent: its `_update` body (ppo.py:113-139, restated
below as test scaffolding: CPU tensors, the :126-127 normalisation, the
randperm loop) calls the patched `_advantages` and `_update_batch`.  One
update from identical CPU networks must match oracle.reference_update: the
advantages bit for bit (rewards of 1.0 and 0.5 are exact in fp32), the
parameters within 2e-5 (the loss gradient comes from the fused kernel)."""

import copy
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from torch import nn

from oracle import ppo_oracle as ref
from ppo_amd import reference_patch
from ppo_amd.agent import PPOConfig, TrainingConfig

pytestmark = pytest.mark.gpu


class ReferenceShapedAgent:
    """The attributes ppo.py:38-59 sets and the `_update` of ppo.py:113-139."""

    def __init__(self, policy, value, config, ppo_config):
        self.config, self.ppo_config = config, ppo_config
        self.policy, self.value = policy, value
        self.parameters = list(policy.parameters()) + list(value.parameters())
        self.optimizer = torch.optim.Adam(self.parameters, lr=config.lr)
        self.rollout = []

    def _update(self):
        observations = torch.as_tensor(
            np.array([s.transition.observation for s in self.rollout]), dtype=torch.float32)
        actions = torch.as_tensor([s.transition.action for s in self.rollout],
                                  dtype=torch.int64)
        old_log_probs = torch.stack([s.log_prob for s in self.rollout])
        old_values = torch.stack([s.value for s in self.rollout])
        advantages = self._advantages(old_values)
        returns = advantages + old_values
        if len(advantages) > 1:
            advantages = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
        for _ in range(self.ppo_config.epochs):
            indices = torch.randperm(len(actions))
            for start in range(0, len(actions), self.config.batch_size):
                b = indices[start : start + self.config.batch_size]
                self._update_batch(observations[b], actions[b], old_log_probs[b],
                                   advantages[b], returns[b])


@pytest.mark.parametrize("T", [1, 45, 300])
def test_patched_methods_match_reference_update(dev, T):
    print(f"reference patch T={T}", flush=True)
    torch.manual_seed(24)
    policy, value = ref.reference_mlp(4, 64, 2), ref.reference_mlp(4, 64, 1)
    config = TrainingConfig(hidden_size=64, batch_size=32)
    cls = reference_patch.apply(type("Patched", (ReferenceShapedAgent,), {}))
    agent = cls(copy.deepcopy(policy), copy.deepcopy(value), config, PPOConfig())
    cpu_opt = torch.optim.Adam(list(policy.parameters()) + list(value.parameters()),
                               lr=config.lr)
    g = torch.Generator().manual_seed(T)
    obs = (torch.rand(T, 4, generator=g) - 0.5) * 0.1
    with torch.no_grad():
        logits = policy(obs)
        acts = torch.multinomial(torch.softmax(logits, -1), 1, generator=g).squeeze(1)
        lps = torch.log_softmax(logits, -1).gather(1, acts[:, None]).squeeze(1)
        vals = value(obs).squeeze(1)
    rewards = [1.0 if t % 3 else 0.5 for t in range(T)]
    dones = [t == T - 1 or t == T // 2 for t in range(T)]
    agent.rollout = [SimpleNamespace(
        transition=SimpleNamespace(observation=obs[t].numpy(), action=int(acts[t]),
                                   reward=rewards[t], terminated=dones[t], truncated=False),
        log_prob=lps[t], value=vals[t]) for t in range(T)]

    adv = agent._advantages(vals)
    assert adv.device.type == "cpu" and adv.dtype == torch.float32
    want = torch.tensor(ref.advantages_python(rewards, dones, [float(v) for v in vals],
                                              config.gamma, 0.95), dtype=torch.float32)
    assert torch.equal(adv, want)

    torch.manual_seed(77)
    agent._update()
    torch.manual_seed(77)
    ref.reference_update(policy, value, cpu_opt, obs, acts, lps, vals, rewards, dones,
                         ref.OracleConfig(batch_size=config.batch_size))
    for a, b in zip(agent.parameters, list(policy.parameters()) + list(value.parameters())):
        assert a.device.type == "cpu"
        torch.testing.assert_close(a.detach(), b.detach(), rtol=0, atol=2e-5)
