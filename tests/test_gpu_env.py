"""Vectorised CartPole-v1 on the GPU (ppo_cartpole_step / CartPoleVec) against
the fp64 restatement oracle.cartpole_step_reference (gymnasium's equations;
gymnasium is not installed, so parity with it is unpinned), and an
end-to-end PPO training run entirely on the device.

Tolerance: the kernel evaluates the same fp64 operations in the same order
without contraction; sin/cos of the device library may differ from the
host's by an ulp, so states are compared at rel 1e-14 (abs 1e-16),
observations within 1 fp32 ulp, and done / terminated / step counters
exactly (test states keep clear of the thresholds by > 1e-9)."""

import math

import numpy as np
import pytest
import torch

import ppo_amd
from ppo_amd import _lib
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu


def _kernel_step(dev, state, actions, steps, u, max_steps=500):
    N = state.shape[0]
    st = torch.from_numpy(state).to(dev)
    sp = torch.from_numpy(steps.astype(np.int32)).to(dev)
    ac = torch.from_numpy(actions.astype(np.int32)).to(dev)
    uu = torch.from_numpy(u.astype(np.float32)).to(dev)
    obs = torch.empty(N, 4, device=dev)
    rew = torch.empty(N, device=dev)
    done = torch.empty(N, dtype=torch.uint8, device=dev)
    term = torch.empty(N, dtype=torch.uint8, device=dev)
    rc = _lib.load().ppo_cartpole_step(st.data_ptr(), sp.data_ptr(), ac.data_ptr(), uu.data_ptr(),
                                       max_steps, obs.data_ptr(), rew.data_ptr(), done.data_ptr(),
                                       term.data_ptr(), None, None, None, N,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return (st.cpu().numpy(), obs.cpu().numpy(), rew.cpu().numpy(), done.cpu().numpy(),
            term.cpu().numpy(), sp.cpu().numpy())


def test_cartpole_step_matches_oracle(dev):
    g = np.random.default_rng(7)
    N = 4096
    th = 12 * 2 * math.pi / 360
    state = np.stack([g.uniform(-2.5, 2.5, N), g.uniform(-3, 3, N), g.uniform(-0.25, 0.25, N),
                      g.uniform(-3, 3, N)], axis=1)
    actions = g.integers(0, 2, N)
    steps = g.integers(0, 500, N)
    steps[:16] = 499
    u = g.random((N, 4))
    # keep clear of the thresholds (decisions must not hinge on an ulp)
    nx = state[:, 0] + 0.02 * state[:, 1]
    nth = state[:, 2] + 0.02 * state[:, 3]
    keep = (np.abs(np.abs(nx) - 2.4) > 1e-6) & (np.abs(np.abs(nth) - th) > 1e-6)
    state, actions, steps, u = state[keep], actions[keep], steps[keep], u[keep]
    got = _kernel_step(dev, state, actions, steps, u)
    exp = ref.cartpole_step_reference(state, actions, steps, u.astype(np.float32))
    np.testing.assert_allclose(got[0], exp[0], rtol=1e-14, atol=1e-16)
    ulp = np.abs(got[1].view(np.int32).astype(np.int64) - exp[1].view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    for k in (2, 3, 4, 5):
        np.testing.assert_array_equal(got[k], exp[k])
    assert exp[3].any() and not exp[3].all()  # both outcomes exercised
    assert exp[4].any() and (exp[3] & ~exp[4]).any()  # terminations and truncations


def test_cartpole_vec_reset_and_episode_tally(dev):
    env = ppo_amd.CartPoleVec(256, dev, seed=5)
    obs = env.reset()
    assert obs.shape == (256, 4) and float(obs.abs().max()) <= 0.05
    assert env.observation_space.shape == (4,) and env.action_space.n == 2
    # always pushing right ends every episode early; count dones on the host
    right = torch.ones(256, dtype=torch.int32, device=dev)
    done_total, length = 0, torch.zeros(256, dtype=torch.int64)
    lengths = []
    for _ in range(60):
        _, r, d, term = env.step(right)
        assert torch.all(r == 1.0)
        dd = d.cpu().bool()
        length += 1
        lengths += length[dd].tolist()
        length[dd] = 0
        done_total += int(dd.sum())
    count, mean_return = env.episode_stats()
    assert count == done_total == len(lengths) > 0
    assert mean_return == pytest.approx(sum(lengths) / len(lengths), rel=1e-6)
    assert env.episode_stats()[0] == 0  # the tally restarts


def test_ppo_trains_cartpole_on_device(dev):
    """PPO (configuration 1's networks: 4-64-64 tanh) on 64 vectorised
    CartPole-v1 environments, every step on the GPU: the mean return of
    completed episodes rises from ~20 (random play) past 300 within 30
    iterations of 128 steps."""
    from ppo_amd.train_cartpole import train

    recs = train(num_envs=64, steps=128, iterations=30, seed=24, device=str(dev))
    first = recs[0]["mean_return"]
    best = max(r["mean_return"] for r in recs if r["episodes"] > 0)
    print(f"cartpole: first {first:.1f}, best {best:.1f}", flush=True)
    assert first < 40 and best > 300


def test_graphed_collection_matches_eager_steps(dev):
    """VecPPO.collect replayed from one HIP graph fills the buffer exactly as
    the same kernels run step by step on the same uniforms (max_steps 20, so
    truncation resets read the reset uniforms), across the eager warm-up,
    the capture and two replays."""
    from ppo_amd.agent import MLP

    torch.manual_seed(3)
    T, N = 24, 96
    policy, value = MLP(4, 64, 2, "tanh").to(dev), MLP(4, 64, 1, "tanh").to(dev)
    vec = ppo_amd.VecPPO(policy, value, graphs=True)
    env_a = ppo_amd.CartPoleVec(N, device=dev, seed=9, max_steps=20)
    env_b = ppo_amd.CartPoleVec(N, device=dev, seed=9, max_steps=20)
    buf_a = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    buf_b = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    obs_a, obs_b = env_a.reset().clone(), env_b.reset().clone()
    gen = torch.Generator(device=dev).manual_seed(1)
    for it in range(4):
        obs_a = vec.collect(env_a, buf_a, obs_a, generator=gen, fused=False)
        plan = next(iter(vec._collect_plans.values()))
        assert (plan.graph is not None) == (it >= 1)
        ua, ur = plan.uact.clone(), plan.ureset.clone()
        buf_b.reset()
        o = obs_b
        for t in range(T):
            acts, _, _ = vec.act(o, buffer=buf_b, uniforms=ua[t].contiguous())
            o = env_b.step_into(acts, buf_b.rewards[t], buf_b.dones[t],
                                reset_uniforms=ur[t].contiguous())
            buf_b.step += 1
        obs_b = o.clone()
        buf_b.finish(vec.value(obs_b).reshape(-1))
        assert torch.equal(obs_a, obs_b), it
        for name in ("observations", "actions", "log_probs", "values", "rewards", "dones",
                     "last_value"):
            assert torch.equal(getattr(buf_a, name), getattr(buf_b, name)), (it, name)
        assert buf_a.step == buf_b.step == T
        assert int(buf_a.dones.sum()) > 0
    assert env_a.episode_stats() == env_b.episode_stats()


@pytest.mark.parametrize("N,H,act", [(96, 64, "tanh"), (37, 32, "relu"), (5, 128, "tanh")])
def test_fused_rollout_matches_step_by_step(dev, N, H, act):
    """ppo_cartpole_rollout_f32 (the whole rollout in one launch) fills the
    buffer, advances the environments and keeps the episode tally exactly as
    the per-step act + step launches do on the same uniforms (max_steps 20:
    truncation resets included; ragged N)."""
    from ppo_amd.agent import MLP

    torch.manual_seed(4)
    T = 24
    policy, value = MLP(4, H, 2, act).to(dev), MLP(4, H, 1, act).to(dev)
    vec = ppo_amd.VecPPO(policy, value, graphs=True)
    envs = [ppo_amd.CartPoleVec(N, device=dev, seed=9, max_steps=20) for _ in range(2)]
    # "cuda" without an index, as train_cartpole passes it
    bufs = [ppo_amd.RolloutBuffer(T, N, (4,), device="cuda") for _ in range(2)]
    obs = [e.reset().clone() for e in envs]
    gens = [torch.Generator(device=dev).manual_seed(1) for _ in range(2)]
    for it in range(3):
        obs[0] = vec.collect(envs[0], bufs[0], obs[0], generator=gens[0], fused=True)
        obs[1] = vec.collect(envs[1], bufs[1], obs[1], generator=gens[1], fused=False)
        assert torch.equal(obs[0], obs[1]), it
        for name in ("observations", "actions", "log_probs", "values", "rewards", "dones",
                     "last_value"):
            assert torch.equal(getattr(bufs[0], name), getattr(bufs[1], name)), (it, name)
        for name in ("state", "steps", "obs", "_ret", "_done_sum", "_done_count"):
            assert torch.equal(getattr(envs[0], name), getattr(envs[1], name)), (it, name)
        assert bufs[0].step == T and int(bufs[0].dones.sum()) > 0
    assert envs[0].episode_stats() == envs[1].episode_stats()


def test_fused_rollout_rejects_other_shapes(dev):
    from ppo_amd.agent import MLP

    policy, value = MLP(6, 32, 3, "tanh").to(dev), MLP(6, 32, 1, "tanh").to(dev)
    vec = ppo_amd.VecPPO(policy, value)
    env = ppo_amd.CartPoleVec(8, device=dev)
    buf = ppo_amd.RolloutBuffer(4, 8, (4,), device=dev)
    with pytest.raises(ValueError):
        vec.collect(env, buf, env.reset().clone(), fused=True)
