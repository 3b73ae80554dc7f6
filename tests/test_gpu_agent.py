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


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("T,activation", [(37, "relu"), (200, "tanh")])
def test_agent_update_matches_reference(dev, T, activation, fused):
    config = TrainingConfig(hidden_size=64, batch_size=32)
    agent = PPOAgent(cartpole_like(), config, device=dev, activation=activation,
                     fused_update=fused)
    assert agent.fused_update == fused
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


# ---------------------------------------------------------------------------
# The drop-in agent driven the way the reference's runner drives it
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("fused,atol", [(True, 2e-5), (False, 1e-6)])
def test_agent_drives_like_reference_runner(dev, fused, atol):
    """rl/deep/tests/test_runner.py:9-25 for the GPU agent: 16 training
    episodes and 4 evaluation episodes of single-env CartPole through
    start_episode / select_action / update / end_episode (runner.py:42-84),
    with the test's config (hidden 16, batch 4, seed 24) and its assertions.
    The same episodes are then run by the CPU restatement of the reference
    agent (oracle.ReferenceAgent) from the same seed: both consume the global
    CPU generator identically (Categorical sampling, torch.randperm), so the
    trajectories agree step for step and the parameters to fp32 noise
    (the fused update sums gradients in another order than torch and
    applies Adam in one kernel: 2e-5; torch's MLPs + the fused loss: 1e-6).""" 
    config = TrainingConfig(batch_size=4, warmup_steps=4, hidden_size=16, seed=24)
    print("runner-style: GPU agent", flush=True)
    env = ref.CartPoleHost()
    agent = PPOAgent(env, config, device=dev, fused_update=fused)
    assert agent.fused_update == fused
    train = [ref.run_episode(env, agent, ep, config.seed, training=True) for ep in range(16)]
    evals = [ref.run_episode(ref.CartPoleHost(), agent, ep, config.seed, training=False)
             for ep in range(4)]
    assert train[0][2] or train[0][3]
    assert np.mean([e[0] for e in evals]) >= 8
    term = np.mean([e[2] for e in evals])
    success = np.mean([e[3] for e in evals])
    assert term + success == 1.0

    print("runner-style: CPU reference agent", flush=True)
    cpu_env = ref.CartPoleHost()
    cpu = ref.ReferenceAgent(hidden_size=16, batch_size=4, seed=24)
    cpu_train = [ref.run_episode(cpu_env, cpu, ep, 24, training=True) for ep in range(16)]
    cpu_evals = [ref.run_episode(ref.CartPoleHost(), cpu, ep, 24, training=False)
                 for ep in range(4)]
    assert [t[:2] for t in train] == [t[:2] for t in cpu_train]
    assert [t[:2] for t in evals] == [t[:2] for t in cpu_evals]
    cpu_params = list(cpu.policy.parameters()) + list(cpu.value.parameters())
    worst = max(float((a.detach().cpu() - b.detach()).abs().max())
                for a, b in zip(agent.parameters, cpu_params))
    print(f"  {sum(t[1] for t in train)} training steps; max |param diff| {worst:.2e}",
          flush=True)
    for a, b in zip(agent.parameters, cpu_params):
        torch.testing.assert_close(a.detach().cpu(), b.detach(), rtol=0, atol=atol)


def test_agent_minibatch_indices_follow_randperm(dev, monkeypatch):
    """ppo.py:129-139: the rows _update hands to _update_batch are the slices
    of torch.randperm drawn on the global CPU generator, epoch by epoch, bit
    for bit.  Each step's observation carries its own index."""
    T, B = 30, 7
    config = TrainingConfig(hidden_size=16, batch_size=B)
    agent = PPOAgent(cartpole_like(), config, device=dev)
    agent.rollout = [
        _rollout_step(1.0, t == T - 1, np.array([t, 0, 0, 0], np.float32), t % 2, -0.7, 0.1)
        for t in range(T)
    ]
    seen = []
    monkeypatch.setattr(agent, "_update_batch",
                        lambda obs, *a, **k: seen.append(obs[:, 0].cpu().to(torch.int64)))
    torch.manual_seed(99)
    agent._update()
    torch.manual_seed(99)
    expected = []
    for _ in range(agent.ppo_config.epochs):
        idx = torch.randperm(T)
        expected += [idx[s : s + B] for s in range(0, T, B)]
    assert len(seen) == len(expected)
    for a, b in zip(seen, expected):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,B", [(30, 7), (500, 128)])
def test_fused_agent_minibatch_indices_follow_randperm(dev, monkeypatch, T, B):
    """The fused loop draws every epoch's torch.randperm before the first
    minibatch and slices them on the device: the rows of each minibatch are
    still the reference's slices, bit for bit, and the loop consumes the
    global generator exactly as ppo.py:129-131 does (the next draw after the
    update is the same)."""
    config = TrainingConfig(hidden_size=16, batch_size=B)
    agent = PPOAgent(cartpole_like(), config, device=dev)
    assert agent.fused_update
    agent.rollout = [
        _rollout_step(1.0, t == T - 1, np.array([t, 0, 0, 0], np.float32), t % 2, -0.7, 0.1)
        for t in range(T)
    ]
    seen = []
    monkeypatch.setattr(agent._vec, "_minibatch",
                        lambda idx, arrays: seen.append(idx.cpu().clone()) or {})
    torch.manual_seed(99)
    agent._update()
    after = torch.randint(0, 1 << 30, (4,))
    torch.manual_seed(99)
    expected = []
    for _ in range(agent.ppo_config.epochs):
        idx = torch.randperm(T)
        expected += [idx[s : s + B] for s in range(0, T, B)]
    assert torch.equal(after, torch.randint(0, 1 << 30, (4,)))
    assert len(seen) == len(expected)
    for a, b in zip(seen, expected):
        assert torch.equal(a, b)


def test_fused_agent_repeated_lengths_replay_graphs(dev):
    """Episodes of the previous episode's length replay the captured update
    (graphs): two agents from one seed, one with graphs and one without,
    stay identical bit for bit over episodes of lengths 40, 40, 40, 17, 40."""
    config = TrainingConfig(hidden_size=32, batch_size=16)
    agents = [PPOAgent(cartpole_like(), config, device=dev) for _ in range(2)]
    agents[1].graphs = False  # (same optimizer kind: a device step counter)
    g = torch.Generator().manual_seed(8)
    for ep, T in enumerate([40, 40, 40, 17, 40]):
        obs = (torch.rand(T, 4, generator=g) - 0.5) * 0.1
        acts = torch.randint(0, 2, (T,), generator=g)
        lps = -0.69 + 0.05 * torch.randn(T, generator=g)
        vals = torch.randn(T, generator=g)
        for agent in agents:
            agent.rollout = [_rollout_step(1.0, t == T - 1, obs[t].numpy(), int(acts[t]),
                                           float(lps[t]), float(vals[t])) for t in range(T)]
            torch.manual_seed(100 + ep)
            agent._update()
        torch.cuda.synchronize()
        for a, b in zip(agents[0].parameters, agents[1].parameters):
            assert torch.equal(a, b), ep
    assert agents[0]._vec.update_graphed_ready()


def test_select_action_one_copy_matches_torch_forward(dev):
    """select_action's fused forward (both networks in one launch, logits and
    value in one buffer) gives torch's forward within fp32 noise, and the
    same draw from the global generator."""
    config = TrainingConfig(hidden_size=128)
    agent = PPOAgent(cartpole_like(), config, device=dev)
    g = torch.Generator().manual_seed(2)
    for k in range(20):
        o = ((torch.rand(4, generator=g) - 0.5) * 0.2).numpy()
        torch.manual_seed(k)
        a = agent.select_action(o)
        step = agent.pending_step
        with torch.no_grad():
            x = torch.as_tensor(o).to(dev)
            logits = agent.policy(x).cpu()
            value = agent.value(x).squeeze().cpu()
        torch.manual_seed(k)
        dist = torch.distributions.Categorical(logits=logits)
        assert int(dist.sample()) == a
        torch.testing.assert_close(step.log_prob, dist.log_prob(torch.tensor(a)),
                                   rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(step.value, value, rtol=1e-5, atol=1e-6)
        assert step.value.dim() == 0 and step.log_prob.dim() == 0
        assert agent.select_action(o, training=False) == int(torch.argmax(logits))


def test_agent_rejects_out_of_range_actions_without_syncing(dev):
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=16), device=dev)
    agent.rollout = [_rollout_step(1.0, False, action=0), _rollout_step(1.0, True, action=2)]
    with pytest.raises(ValueError, match="support"):
        agent._update()


def test_agent_advantages_with_non_representable_rewards(dev):
    """Rewards that fp32 cannot hold (0.1, 0.3, ...) enter the kernel rounded
    to fp32: the advantages stay within max|r| * 2^-24 / (1 - gamma*lambda)
    (plus one fp32 ulp of the result) of the reference's Python-float loop
    (ppo.py:173-193), the bound PPOAgent._advantages states."""
    config = TrainingConfig(hidden_size=16)
    pcfg = PPOConfig()
    agent = PPOAgent(cartpole_like(), config, pcfg, device=dev)
    g = torch.Generator().manual_seed(3)
    T = 500
    rewards = [round(0.1 * int(k), 1) for k in torch.randint(-9, 10, (T,), generator=g)]
    values = torch.randn(T, generator=g)
    dones = [bool(x) for x in (torch.rand(T, generator=g) < 0.02)] + [True]
    dones = dones[:T]
    agent.rollout = [_rollout_step(r, dn, value=float(v)) for r, dn, v in zip(rewards, dones, values)]
    got = agent._advantages(values).cpu().double()
    want = torch.tensor(ref.advantages_python(rewards, dones, [float(v) for v in values],
                                              config.gamma, pcfg.gae_lambda), dtype=torch.float64)
    bound = max(abs(r) for r in rewards) * 2.0**-24 / (1 - config.gamma * pcfg.gae_lambda)
    ulp = want.abs() * 2.0**-23
    err = (got - want).abs()
    print(f"  max |adv - reference| {float(err.max()):.2e} (bound {bound:.2e})", flush=True)
    assert bool((err <= bound + ulp).all())


@pytest.mark.parametrize("fused", [True, False])
def test_agent_vf_clip_uses_rollout_values(dev, monkeypatch, fused):
    """PPOConfig.vf_clip (a field the reference does not have) carries the
    rollout's values into _update_batch: one minibatch's raw gradients match
    update_batch_grads_reference with value clipping; without the old values
    _update_batch refuses."""
    T, H = 64, 32
    config = TrainingConfig(hidden_size=H, batch_size=T)
    pcfg = PPOConfig(vf_clip=0.2, gradient_clip=1e9)
    agent = PPOAgent(cartpole_like(), config, pcfg, device=dev, fused_update=fused)
    cpu_policy = copy.deepcopy(agent.policy).cpu()
    cpu_value = copy.deepcopy(agent.value).cpu()
    g = torch.Generator().manual_seed(4)
    obs = torch.randn(T, 4, generator=g)
    acts = torch.randint(0, 2, (T,), generator=g)
    lps = -torch.rand(T, generator=g)
    adv = torch.randn(T, generator=g)
    ret = torch.randn(T, generator=g)
    with torch.no_grad():
        old_v = cpu_value(obs).squeeze(1) + 0.3 * torch.randn(T, generator=g)
    monkeypatch.setattr(agent.optimizer, "step", lambda: None)
    with pytest.raises(ValueError, match="old_values"):
        agent._update_batch(obs.to(dev), acts.to(dev), lps.to(dev), adv.to(dev), ret.to(dev))
    agent._update_batch(obs.to(dev), acts.to(dev), lps.to(dev), adv.to(dev), ret.to(dev),
                        old_values=old_v.to(dev))
    o = ref.update_batch_grads_reference(cpu_policy, cpu_value, obs, acts, lps, adv, ret,
                                         old_values=old_v, vf_clip=0.2)
    for p, gref in zip(agent.parameters, o["grads"]):
        torch.testing.assert_close(p.grad.cpu(), gref, rtol=1e-4, atol=1e-5 * float(gref.abs().max()))
    # and a whole _update runs with vf_clip set
    agent.rollout = [_rollout_step(1.0, t == 19, value=0.1 * t) for t in range(20)]
    agent._update()


# ---------------------------------------------------------------------------
# Configuration 1 at its own shape: T=128 x N=8, 4-64-64 tanh, minibatches
# of 256, 4 epochs, through every VecPPO update path, against the CPU oracle
# (two rollouts in a row, so the graph path replays captured graphs).
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mode", ["unfused", "fused_mlp", "graphs"])
def test_vec_update_config1_matches_reference(dev, mode):
    T, N, H, MB = 128, 8, 64, 256
    torch.manual_seed(24)
    policy = MLP(4, H, 2, "tanh")
    value = MLP(4, H, 1, "tanh")
    cpu_policy, cpu_value = copy.deepcopy(policy), copy.deepcopy(value)
    cpu_opt = torch.optim.Adam(list(cpu_policy.parameters()) + list(cpu_value.parameters()),
                               lr=3e-4)
    kw = {"unfused": dict(fused_update=False),
          "fused_mlp": dict(fused_mlp=True),
          "graphs": dict(fused_mlp=True, graphs=True)}[mode]
    vec = ppo_amd.VecPPO(policy.to(dev), value.to(dev), PPOConfig(), gamma=0.99, lr=3e-4,
                         batch_size=MB, generator=torch.Generator().manual_seed(7), **kw)
    cpu_gen = torch.Generator().manual_seed(7)
    buf = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    for rollout in range(2):
        print(f"config1 mode={mode} rollout={rollout}", flush=True)
        g = torch.Generator().manual_seed(50 + rollout)
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
        buf.reset()
        for t in range(T):
            buf.add(obs[t].to(dev), acts[t].to(torch.int32).to(dev), rewards[t].to(dev),
                    dones[t].to(dev), vals[t].to(dev), lps[t].to(dev))
        buf.finish(last_v.to(dev))
        vec.update(buf)
        torch.cuda.synchronize()

        adv, ret = ref.gae_numpy(rewards.numpy(), vals.numpy(), dones.numpy(), last_v.numpy(),
                                 0.99, 0.95)
        adv_n = ref.normalize_reference(torch.from_numpy(adv).reshape(-1))
        ref.reference_epochs(cpu_policy, cpu_value, cpu_opt, obs.reshape(-1, 4),
                             acts.reshape(-1), lps.reshape(-1), adv_n,
                             torch.from_numpy(ret).reshape(-1),
                             ref.OracleConfig(batch_size=MB), generator=cpu_gen)
        cpu_params = list(cpu_policy.parameters()) + list(cpu_value.parameters())
        worst = max(float((a.detach().cpu() - b.detach()).abs().max())
                    for a, b in zip(vec.parameters, cpu_params))
        print(f"  max |param diff| {worst:.2e}", flush=True)
        for a, b in zip(vec.parameters, cpu_params):
            torch.testing.assert_close(a.detach().cpu(), b.detach(), rtol=0, atol=2e-5)
    if mode == "graphs":
        assert vec.update_graphed_ready()


@pytest.mark.parametrize("H,A,act", [(128, 2, "relu"), (64, 18, "tanh"), (16, 5, "relu")])
def test_mlp_forward_categorical_matches_torch(dev, H, A, act):
    """ppo_mlp_forward_cat_f32 on device tensors (N rows) and on pinned host
    memory (one row, the path select_action takes): torch's forward of both
    networks within fp32 noise."""
    torch.manual_seed(H + A)
    pol, val = MLP(6, H, A, act).to(dev), MLP(6, H, 1, act).to(dev)
    obs = torch.randn(1000, 6, device=dev)
    logits, values = ppo_amd.mlp_forward_categorical(pol, val, obs)
    with torch.no_grad():
        torch.testing.assert_close(logits, pol(obs), rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(values, val(obs).squeeze(1), rtol=1e-5, atol=1e-5)
    io = torch.zeros(6 + A + 1, dtype=torch.float32, pin_memory=True)
    io[:6] = obs[7].cpu()
    lo, vo = io[6:6 + A].view(1, A), io[6 + A:]
    ppo_amd.mlp_forward_categorical(pol, val, io[:6].view(1, 6), logits_out=lo, values_out=vo)
    torch.cuda.synchronize(dev)
    # (the one-row launch runs the one-workgroup form, whose arithmetic is
    # the many-row form's step for step)
    assert torch.equal(lo[0], logits[7].cpu()) and torch.equal(vo[0], values[7].cpu())


@pytest.mark.parametrize("D,H,A,act", [(4, 128, 2, "relu"), (64, 128, 32, "tanh"),
                                       (6, 64, 18, "relu"), (5, 32, 17, "tanh"),
                                       (3, 16, 1, "relu")])
def test_act_one_workgroup_form_matches_many_row_form(dev, D, H, A, act):
    """Launches of at most 16 rows (one workgroup, weights loaded up front)
    give the rows of a 40-row launch bit for bit: logits and values of
    ppo_mlp_forward_cat_f32, actions, log-probabilities and values of
    ppo_mlp_act_cat_f32 (the same uniforms)."""
    print(f"act forms D={D} H={H} A={A} {act}", flush=True)
    torch.manual_seed(D * H + A)
    pol, val = MLP(D, H, A, act).to(dev), MLP(D, H, 1, act).to(dev)
    obs = torch.randn(40, D, device=dev)
    u = torch.rand(40, device=dev)
    logits, values = ppo_amd.mlp_forward_categorical(pol, val, obs)
    acts, lps, vals = ppo_amd.mlp_act_categorical(pol, val, obs, uniforms=u)
    for lo, hi in ((0, 16), (16, 17), (23, 40 - 11)):
        l2, v2 = ppo_amd.mlp_forward_categorical(pol, val, obs[lo:hi].contiguous())
        a2, p2, w2 = ppo_amd.mlp_act_categorical(pol, val, obs[lo:hi].contiguous(),
                                                 uniforms=u[lo:hi].contiguous())
        assert torch.equal(l2, logits[lo:hi]) and torch.equal(v2, values[lo:hi])
        assert torch.equal(a2, acts[lo:hi]) and torch.equal(p2, lps[lo:hi])
        assert torch.equal(w2, vals[lo:hi])
    with torch.no_grad():
        torch.testing.assert_close(logits, pol(obs), rtol=1e-5, atol=1e-5)


def test_select_action_after_network_replaced(dev):
    """A network object replaced by one the fused forward does not run
    (here: a GELU MLP) makes select_action fall back to torch's forward."""
    agent = PPOAgent(cartpole_like(), TrainingConfig(hidden_size=32), device=dev)
    o = np.zeros(4, np.float32)
    agent.select_action(o)
    agent.policy = torch.nn.Sequential(torch.nn.Linear(4, 32), torch.nn.GELU(),
                                       torch.nn.Linear(32, 2)).to(dev)
    torch.manual_seed(3)
    a = agent.select_action(o)
    with torch.no_grad():
        logits = agent.policy(torch.as_tensor(o).to(dev)).cpu()
    torch.manual_seed(3)
    assert a == int(torch.distributions.Categorical(logits=logits).sample())
