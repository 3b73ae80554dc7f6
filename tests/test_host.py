"""Host-side logic that needs no GPU: the reference-mirroring surface
(configs, records, cartpole_sizes, rollout storage) and the ops' argument
validation, which must raise rather than fall back to the CPU."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import ppo_amd
from ppo_amd.agent import PPOAgent, PPOConfig, TrainingConfig


def cartpole_like():
    return SimpleNamespace(observation_space=SimpleNamespace(shape=(4,)),
                           action_space=SimpleNamespace(n=2))


def test_config_defaults_match_reference():
    # rl/deep/type.py:30-41 and rl/deep/agents/ppo.py:15-22
    t = TrainingConfig()
    assert (t.gamma, t.lr, t.seed, t.hidden_size, t.batch_size) == (0.99, 3e-4, 24, 128, 128)
    p = PPOConfig()
    assert (p.epochs, p.clip_ratio, p.gae_lambda, p.value_coef, p.entropy_coef,
            p.gradient_clip, p.vf_clip) == (4, 0.2, 0.95, 0.5, 0.01, 0.5, None)


def test_cartpole_sizes_errors():
    assert ppo_amd.cartpole_sizes(cartpole_like()) == (4, 2)
    with pytest.raises(TypeError, match="Box"):
        ppo_amd.cartpole_sizes(SimpleNamespace(observation_space=None,
                                               action_space=SimpleNamespace(n=2)))
    with pytest.raises(TypeError, match="Discrete"):
        ppo_amd.cartpole_sizes(SimpleNamespace(observation_space=SimpleNamespace(shape=(4,)),
                                               action_space=SimpleNamespace(shape=(2,))))


def test_ppo_stores_rollout_step_after_update():
    """rl/deep/tests/test_ppo.py:11-31 (acting needs no kernel)."""
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16, seed=24), device="cpu")
    observation = np.zeros(4, dtype=np.float32)
    action = agent.select_action(observation)
    agent.update(observation, action, reward=1.0, next_observation=np.ones(4, np.float32),
                 terminated=False, truncated=True)
    assert agent.pending_step is None
    assert len(agent.rollout) == 1
    assert agent.rollout[0].transition.truncated
    assert agent.rollout[0].log_prob.shape == torch.Size([])
    assert agent.rollout[0].value.shape == torch.Size([])


def test_agent_init_matches_reference_init():
    """Same seed -> the same initial weights as the reference's CPU MLPs."""
    torch.manual_seed(24)
    pol = ppo_amd.MLP(4, 16, 2)
    val = ppo_amd.MLP(4, 16, 1)
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16), device="cpu")
    for a, b in zip(agent.parameters, list(pol.parameters()) + list(val.parameters())):
        assert torch.equal(a, b)


def test_ops_refuse_cpu_tensors():
    r = torch.zeros(4, 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        ppo_amd.gae(r, r, torch.zeros(4, 2, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="GPU only"):
        ppo_amd.normalize_advantages(torch.zeros(5))
    with pytest.raises(RuntimeError, match="GPU only"):
        ppo_amd.ppo_loss_discrete_fused(torch.zeros(3, 2), torch.zeros(3, dtype=torch.int64),
                                        *[torch.zeros(3)] * 4)


def test_agent_update_on_cpu_raises_not_falls_back():
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16), device="cpu")
    obs = np.zeros(4, np.float32)
    for _ in range(3):
        a = agent.select_action(obs)
        agent.update(obs, a, 1.0, obs, False, False)
    with pytest.raises(RuntimeError, match="GPU only"):
        agent.end_episode()


def test_rollout_buffer_validation():
    with pytest.raises(ValueError):
        ppo_amd.RolloutBuffer(0, 4, (4,), device="cpu")
    buf = ppo_amd.RolloutBuffer(2, 3, (4,), device="cpu")
    z = torch.zeros(3)
    buf.add(torch.zeros(3, 4), torch.zeros(3, dtype=torch.int32), z, z.to(torch.uint8), z, z)
    buf.add(torch.zeros(3, 4), torch.zeros(3, dtype=torch.int32), z, z.to(torch.uint8), z, z)
    with pytest.raises(IndexError):
        buf.add(torch.zeros(3, 4), torch.zeros(3, dtype=torch.int32), z, z.to(torch.uint8), z, z)
    assert buf.observations.shape == (2, 3, 4) and buf.dones.dtype == torch.uint8


def test_vecppo_graph_options_validated():
    from ppo_amd.agent import MLP

    pol, val = MLP(4, 8, 2), MLP(4, 8, 1)
    with pytest.raises(ValueError, match="fused_update"):
        ppo_amd.VecPPO(pol, val, graphs=True, fused_update=False)
    with pytest.raises(ValueError, match="graph_chunk"):
        ppo_amd.VecPPO(pol, val, graphs=True, graph_chunk=0)


def test_sample_categorical_matches_torch_distribution():
    """agent.sample_categorical draws the action a Categorical(logits) draws
    from the same global-generator state, returns its log_prob bit for bit,
    and leaves the generator in the same state (ppo.py:72-78)."""
    from torch.distributions import Categorical

    from ppo_amd.agent import sample_categorical

    g = torch.Generator().manual_seed(3)
    cases = [torch.randn(A, generator=g) * s for A in (1, 2, 3, 18) for s in (1e-3, 1.0, 40.0)
             for _ in range(30)]
    cases += [torch.tensor([0.0, float("-inf")]), torch.tensor([-1e30, 0.0, 1e30])]
    for k, logits in enumerate(cases):
        torch.manual_seed(k)
        dist = Categorical(logits=logits)
        a_ref = dist.sample()
        lp_ref = dist.log_prob(a_ref)
        state_ref = torch.get_rng_state()
        torch.manual_seed(k)
        a, lp = sample_categorical(logits)
        assert a == int(a_ref) and lp.dim() == 0 and lp.dtype == torch.float32
        assert torch.equal(lp, lp_ref), (k, lp, lp_ref)
        assert torch.equal(torch.get_rng_state(), state_ref)


def test_sample_categorical_rejects_nan_logits_like_the_distribution():
    from torch.distributions import Categorical

    from ppo_amd.agent import sample_categorical

    bad = torch.tensor([0.5, float("nan")])
    with pytest.raises(ValueError):
        Categorical(logits=bad)
    with pytest.raises(ValueError):
        sample_categorical(bad)


def _steps(n, obs_dim=4, shape=()):
    from ppo_amd.agent import RolloutStep, Transition

    g = torch.Generator().manual_seed(n)
    out = []
    for t in range(n):
        obs = torch.rand(obs_dim, generator=g).numpy().astype(np.float64)
        tr = Transition(observation=obs, action=int(t % 2), reward=0.5 * t,
                        next_observation=obs, terminated=t == n - 1, truncated=t == n // 2)
        out.append(RolloutStep(tr, log_prob=torch.randn(shape, generator=g),
                               value=torch.randn(shape, generator=g)))
    return out


@pytest.mark.parametrize("n,shape", [(1, ()), (37, ()), (37, (1,)), (500, ())])
def test_upload_rollout_packs_every_array(n, shape):
    """PPOAgent._upload_rollout (one pinned buffer, one copy; on a CPU agent
    the same packing into host memory) holds ppo.py:114-122's arrays and the
    rewards and done flags :173-193 reads, with the dtypes the kernels take."""
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16), device="cpu")
    agent.rollout = _steps(n, shape=shape)
    st = agent._upload_rollout()
    steps = agent.rollout
    assert st["obs"].dtype == torch.float32 and st["obs"].shape == (n, 4)
    assert torch.equal(st["obs"], torch.as_tensor(
        np.array([s.transition.observation for s in steps]), dtype=torch.float32))
    assert st["act"].dtype == torch.int64
    assert st["act"].tolist() == [s.transition.action for s in steps]
    assert torch.equal(st["lp"], torch.stack([s.log_prob for s in steps]).reshape(n))
    assert torch.equal(st["val"], torch.stack([s.value for s in steps]).reshape(n))
    assert st["rew"].tolist() == [s.transition.reward for s in steps]
    assert st["done"].dtype == torch.uint8
    assert st["done"].tolist() == [int(s.transition.terminated or s.transition.truncated)
                                   for s in steps]
    for a in ("obs", "lp", "val", "rew", "act", "done"):
        assert st[a].data_ptr() % 16 == 0, a
    # a second episode of the same length reuses the same arrays
    agent.rollout = _steps(n, shape=shape)[::-1]
    st2 = agent._upload_rollout()
    assert st2["obs"].data_ptr() == st["obs"].data_ptr()
    assert st2["act"].tolist() == [s.transition.action for s in agent.rollout]


def test_upload_rollout_rejects_out_of_range_actions():
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16), device="cpu")
    steps = _steps(5)
    from ppo_amd.agent import RolloutStep

    steps[3] = RolloutStep(steps[3].transition.__class__(
        **{**steps[3].transition.__dict__, "action": 2}), steps[3].log_prob, steps[3].value)
    agent.rollout = steps
    with pytest.raises(ValueError, match="support"):
        agent._upload_rollout()
