"""Pins the runner-level pieces of the CPU oracle: ReferenceAgent
(rl/deep/agents/ppo.py:38-111), run_episode (rl/deep/runner.py:42-84) and
CartPoleHost (the CartPole-v1 env as the runner drives it).  The GPU agent
test compares the drop-in PPOAgent with these, so a shared off-by-one
(a missing final step, an update after an empty episode, a wrong truncation
step) must fail here first.  CPU only.

What is asserted, against the reference's own control flow:
  - one update per training episode, at its end (ppo.py:109-111), over
    exactly one rollout step per env step including the last
    (runner.py:56-74 calls agent.update before checking termination);
  - the last step's done flag is `terminated or truncated`, earlier ones
    False; an episode of one step updates on one sample;
  - evaluation episodes (training=False) record nothing and update nothing,
    and end_episode with an empty rollout leaves the parameters alone;
  - ReferenceAgent.end_episode equals reference_update on the same tensors
    bit for bit (same global generator state);
  - CartPoleHost: truncation at max_steps only when not terminated, no
    automatic reset, a rational known answer of one step and mirror
    symmetry of the dynamics.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ppo_oracle as ref


class ScriptedEnv:
    """Episodes of fixed lengths: episode k ends after lengths[k] steps,
    terminated or truncated as `kinds[k]` says; observations are the step
    index spread over 4 floats, reward 1.0 per step."""

    class _Space:
        def __init__(self, shape=None, n=None):
            self.shape, self.n = shape, n
            self.seeds = []

        def seed(self, seed=None):
            self.seeds.append(seed)
            return [seed]

    def __init__(self, lengths, kinds):
        self.lengths, self.kinds = list(lengths), list(kinds)
        self.observation_space = self._Space(shape=(4,))
        self.action_space = self._Space(n=2)
        self.episode = -1
        self.t = 0
        self.reset_seeds = []
        self.steps_taken = []

    def _obs(self):
        return np.full(4, 0.01 * self.t, dtype=np.float32)

    def reset(self, seed=None):
        self.reset_seeds.append(seed)
        self.episode += 1
        self.t = 0
        self.steps_taken.append(0)
        return self._obs(), {}

    def step(self, action):
        assert action in (0, 1)
        self.t += 1
        self.steps_taken[-1] += 1
        L, kind = self.lengths[self.episode], self.kinds[self.episode]
        end = self.t >= L
        term = end and kind == "terminated"
        trunc = end and kind == "truncated"
        return self._obs(), 1.0, term, trunc, {}


@pytest.fixture
def recorded_updates(monkeypatch):
    """Records every reference_update call (rollout length, rewards, dones)
    and still runs it."""
    calls = []
    original = ref.reference_update

    def spy(policy, value, optimizer, obs, actions, lps, vals, rewards, dones, config):
        calls.append(dict(n=obs.shape[0], rewards=list(rewards), dones=list(dones),
                          actions=actions.clone(), obs=obs.clone()))
        return original(policy, value, optimizer, obs, actions, lps, vals, rewards, dones,
                        config)

    monkeypatch.setattr(ref, "reference_update", spy)
    return calls


def test_run_episode_updates_once_per_episode_over_every_step(recorded_updates):
    lengths = [7, 5, 1, 3]
    kinds = ["terminated", "truncated", "terminated", "truncated"]
    env = ScriptedEnv(lengths, kinds)
    agent = ref.ReferenceAgent(hidden_size=8, batch_size=4, seed=24)
    results = [ref.run_episode(env, agent, ep, seed=100, training=True)
               for ep in range(len(lengths))]
    assert env.reset_seeds == [100, 101, 102, 103]           # runner.py:52
    assert env.action_space.seeds == [100, 101, 102, 103]    # runner.py:53
    assert env.steps_taken == lengths
    for (ret, length, term, trunc), L, kind in zip(results, lengths, kinds):
        assert (ret, length) == (float(L), L)
        assert (term, trunc) == (kind == "terminated", kind == "truncated")
    assert [c["n"] for c in recorded_updates] == lengths
    for c, L in zip(recorded_updates, lengths):
        assert c["rewards"] == [1.0] * L
        assert c["dones"] == [False] * (L - 1) + [True]
        # observation stored per step is the one the action was chosen on
        expect_obs = np.stack([np.full(4, 0.01 * t, np.float32) for t in range(L)])
        assert np.array_equal(c["obs"].numpy(), expect_obs)
    # end_episode leaves the rollout in place; start_episode clears it (ppo.py:61-63)
    assert len(agent.rollout) == lengths[-1]
    agent.start_episode(len(lengths))
    assert agent.rollout == [] and agent.pending is None


def test_evaluation_episodes_record_and_update_nothing(recorded_updates):
    env = ScriptedEnv([4, 2], ["terminated", "truncated"])
    agent = ref.ReferenceAgent(hidden_size=8, batch_size=4, seed=24)
    before = [p.detach().clone() for p in agent.policy.parameters()]
    for ep in range(2):
        ret, length, _, _ = ref.run_episode(env, agent, ep, seed=0, training=False)
        assert agent.rollout == []
    assert recorded_updates == []
    for a, b in zip(before, agent.policy.parameters()):
        assert torch.equal(a, b)


def test_end_episode_with_empty_rollout_does_nothing(recorded_updates):
    agent = ref.ReferenceAgent(hidden_size=8, batch_size=4, seed=24)
    params = [p.detach().clone() for p in
              list(agent.policy.parameters()) + list(agent.value.parameters())]
    state = torch.get_rng_state()
    agent.start_episode(0)
    agent.end_episode()
    assert recorded_updates == []
    assert torch.equal(state, torch.get_rng_state())  # no randperm drawn
    for a, b in zip(params, list(agent.policy.parameters()) + list(agent.value.parameters())):
        assert torch.equal(a, b)


def test_update_without_pending_step_is_ignored():
    agent = ref.ReferenceAgent(hidden_size=8, batch_size=4, seed=24)
    agent.update(np.zeros(4, np.float32), 0, 1.0, np.zeros(4, np.float32), False, False)
    assert agent.rollout == []
    agent.select_action(np.zeros(4, np.float32))
    agent.update(np.zeros(4, np.float32), 1, 1.0, np.zeros(4, np.float32), False, True)
    agent.update(np.zeros(4, np.float32), 1, 1.0, np.zeros(4, np.float32), False, True)
    assert len(agent.rollout) == 1 and agent.rollout[0][3] is True


@pytest.mark.parametrize("L", [1, 9, 300])
def test_end_episode_equals_reference_update_bit_for_bit(L):
    g = torch.Generator().manual_seed(L)
    obs = torch.rand(L, 4, generator=g) * 0.1 - 0.05
    actions = torch.randint(0, 2, (L,), generator=g)
    lps = -0.69 + 0.05 * torch.randn(L, generator=g)
    vals = torch.randn(L, generator=g)
    rewards = [1.0] * L
    dones = [False] * (L - 1) + [True]
    a = ref.ReferenceAgent(hidden_size=16, batch_size=8, seed=7)
    b = ref.ReferenceAgent(hidden_size=16, batch_size=8, seed=7)
    a.rollout = [(obs[t].numpy(), int(actions[t]), rewards[t], dones[t], lps[t], vals[t])
                 for t in range(L)]
    torch.manual_seed(99)
    a.end_episode()
    torch.manual_seed(99)
    ref.reference_update(b.policy, b.value, b.optimizer, obs, actions, lps, vals, rewards,
                         dones, b.config)
    for x, y in zip(list(a.policy.parameters()) + list(a.value.parameters()),
                    list(b.policy.parameters()) + list(b.value.parameters())):
        assert torch.equal(x, y)
    # and the update moved the parameters (it is not a no-op)
    c = ref.ReferenceAgent(hidden_size=16, batch_size=8, seed=7)
    moved = any(not torch.equal(x, y) for x, y in zip(a.policy.parameters(),
                                                      c.policy.parameters()))
    assert moved


def test_cartpole_host_truncates_only_when_not_terminated():
    env = ref.CartPoleHost(max_steps=5)
    env.reset(seed=3)
    flags = [env.step(t % 2)[2:4] for t in range(5)]
    assert flags[:4] == [(False, False)] * 4
    assert flags[4] == (False, True)
    # no automatic reset: the step count and the state carry on
    assert env.steps == 5
    _, _, term, trunc, _ = env.step(0)
    assert (term, trunc) == (False, True)
    # a terminating step at the limit is terminated, not truncated
    env = ref.CartPoleHost(max_steps=1)
    env.reset(seed=0)
    env.state = np.array([2.39, 1.0, 0.0, 0.0])
    _, r, term, trunc, _ = env.step(1)
    assert (r, term, trunc) == (1.0, True, False)


def test_cartpole_host_reset_is_seeded_and_in_range():
    env = ref.CartPoleHost()
    o1, _ = env.reset(seed=11)
    o2, _ = env.reset(seed=11)
    o3, _ = env.reset(seed=12)
    assert np.array_equal(o1, o2) and not np.array_equal(o1, o3)
    assert o1.dtype == np.float32 and np.all(np.abs(o1) <= 0.05)
    assert env.steps == 0


def test_cartpole_dynamics_known_answer_and_mirror_symmetry():
    # From rest with the force +10: temp = 100/11, thetaacc = -600/41,
    # xacc = 400/41, so after one Euler step of tau = 0.02:
    # x = 0, x_dot = 8/41, theta = 0, theta_dot = -12/41.
    env = ref.CartPoleHost()
    env.reset(seed=0)
    env.state = np.zeros(4)
    obs, _, term, trunc, _ = env.step(1)
    expect = np.array([0.0, 8 / 41, 0.0, -12 / 41])
    np.testing.assert_allclose(env.state, expect, rtol=0, atol=1e-15)
    assert np.array_equal(obs, expect.astype(np.float32)) and not term and not trunc
    rng = np.random.default_rng(5)
    for _ in range(50):
        s = rng.uniform(-0.2, 0.2, size=4)
        a = ref._cartpole_dynamics(s, 1)
        b = ref._cartpole_dynamics(-s, 0)
        assert all(x == -y for x, y in zip(a[:4], b[:4])) and a[4] == b[4]
    # the pole angle limit is 12 degrees
    s = np.array([0.0, 0.0, 12 * 2 * math.pi / 360 + 1e-3, 0.0])
    assert ref._cartpole_dynamics(s, 1)[4]


def test_cartpole_host_matches_vectorised_oracle_step():
    env = ref.CartPoleHost(max_steps=500)
    env.reset(seed=4)
    state = env.state.copy()
    for t in range(40):
        a = t % 3 == 0
        nxt, obs, rew, dones, term, steps = ref.cartpole_step_reference(
            state[None, :], np.array([a]), np.array([t]), np.zeros((1, 4)))
        o, r, te, tr, _ = env.step(int(a))
        if dones[0]:
            assert te
            break
        assert np.array_equal(env.state, nxt[0]) and np.array_equal(o, obs[0])
        state = nxt[0]
