"""GPU parity of the fused minibatch gradient through the actor and critic
MLPs (ppo_mlp_cat_grad_f32: ppo.py:141-169 with common.py:16-28's MLP)
against the CPU oracle update_batch_grads_reference (torch autograd on the
same networks in fp64).

Tolerance: every parameter gradient within rel 1e-4 plus an absolute floor
of 1e-5 x max|g| of that tensor (north star: rel 1e-4 for gradients in fp32;
the floor covers elements that cancel to ~0), loss scalars rel 1e-5 (approx_kl,
a cancellation, 1e-6 absolute).  The kernel computes in fp32 like torch; its
sums over the minibatch run in another order than torch's GEMMs.
"""

import copy

import pytest
import torch

import ppo_amd
from ppo_amd.agent import MLP
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu


def assert_grad_close(got, expect, rtol=1e-4, floor=1e-5):
    got = got.detach().cpu().to(torch.float64)
    expect = expect.detach().cpu().to(torch.float64)
    atol = floor * float(expect.abs().max()) if expect.numel() else 0.0
    torch.testing.assert_close(got, expect, rtol=rtol, atol=atol)


def _case(dev, n, D, H, A, act, seed, act64=False):
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    pol, val = MLP(D, H, A, act), MLP(D, H, 1, act)
    obs = torch.randn(n, D, generator=g)
    with torch.no_grad():
        logits = pol(obs)
        old_logits = logits + 0.1 * torch.randn(n, A, generator=g)
        actions = torch.multinomial(torch.softmax(old_logits, -1), 1, generator=g).squeeze(1)
        old_lp = torch.log_softmax(old_logits, -1).gather(1, actions[:, None]).squeeze(1)
        old_v = val(obs).squeeze(1) + 0.1 * torch.randn(n, generator=g)
    adv = torch.randn(n, generator=g)
    ret = torch.randn(n, generator=g)
    actions = actions if act64 else actions.to(torch.int32)
    cpu = dict(obs=obs, actions=actions, old_lp=old_lp, adv=adv, ret=ret, old_v=old_v)
    gpu = {k: v.to(dev) for k, v in cpu.items()}
    return pol, val, cpu, gpu


def _check(dev, n, D, H, A, act, B, seed, vf_clip=None, act64=False, use_index=True):
    print(f"mlp n={n} D={D} H={H} A={A} act={act} B={B} vf_clip={vf_clip} i64={act64}",
          flush=True)
    pol, val, cpu, gpu = _case(dev, n, D, H, A, act, seed, act64)
    g = torch.Generator().manual_seed(seed + 1)
    idx = torch.randperm(n, generator=g)[:B] if use_index else torch.arange(n)
    pol_d, val_d = copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)
    stats = ppo_amd.ppo_mlp_cat_grads(
        pol_d, val_d, gpu["obs"], gpu["actions"], gpu["old_lp"], gpu["adv"], gpu["ret"],
        gpu["old_v"], idx.to(dev) if use_index else None, 0.2, vf_clip, 0.5, 0.01)
    o = ref.update_batch_grads_reference(
        copy.deepcopy(pol).double(), copy.deepcopy(val).double(), cpu["obs"][idx],
        cpu["actions"][idx], cpu["old_lp"][idx], cpu["adv"][idx], cpu["ret"][idx],
        cpu["old_v"][idx], 0.2, vf_clip, 0.5, 0.01)
    params = list(pol_d.parameters()) + list(val_d.parameters())
    for p, gr in zip(params, o["grads"]):
        assert_grad_close(p.grad, gr)
    for k in ("loss", "policy", "value", "entropy", "clipfrac"):
        assert stats[k].item() == pytest.approx(o[k].item(), rel=1e-5, abs=1e-6), k
    assert stats["approx_kl"].item() == pytest.approx(o["approx_kl"].item(), abs=1e-6)
    return pol_d, val_d, params


@pytest.mark.parametrize(
    "n,D,H,A,act,B",
    [
        (1024, 4, 64, 2, "tanh", 256),     # configuration 1's minibatch
        (1024, 4, 128, 2, "relu", 128),    # the reference's MLP(4, 128, 2) and batch_size
        (300, 8, 32, 5, "relu", 100),      # B not a multiple of 16
        (200, 17, 64, 18, "tanh", 37),     # odd obs dim, 18 actions
        (64, 6, 16, 3, "tanh", 64),        # H = 16
        (5000, 4, 64, 2, "tanh", 4096),    # a large minibatch (256 workgroups)
        (50, 3, 128, 32, "relu", 1),       # one row, the widest action set
        (300, 7, 128, 9, "tanh", 37),      # H = 128 (16-wave workgroups), a partial block
        (5000, 4, 128, 2, "relu", 4096),   # H = 128, 256 row blocks
    ],
)
def test_mlp_grads_match_oracle(dev, n, D, H, A, act, B):
    _check(dev, n, D, H, A, act, B, seed=n + 7 * D + H + A)


def test_mlp_grads_value_clipping_and_int64_actions(dev):
    _check(dev, 512, 4, 64, 2, "tanh", 200, seed=3, vf_clip=0.2, act64=True)


def test_mlp_grads_without_index_uses_all_rows(dev):
    _check(dev, 96, 5, 32, 4, "relu", 96, seed=4, use_index=False)


def test_mlp_grads_match_unfused_gpu_path(dev):
    """The same minibatch through torch's MLPs on the GPU, the fused loss op
    and autograd gives the same gradients."""
    pol, val, cpu, gpu = _case(dev, 512, 4, 64, 2, "tanh", seed=9)
    idx = torch.randperm(512, generator=torch.Generator().manual_seed(10))[:256].to(dev)
    p1, v1 = copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)
    p2, v2 = copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)
    ppo_amd.ppo_mlp_cat_grads(p1, v1, gpu["obs"], gpu["actions"], gpu["old_lp"], gpu["adv"],
                              gpu["ret"], index=idx)
    obs_b = gpu["obs"][idx]
    loss, _ = ppo_amd.ppo_loss_discrete(
        p2(obs_b).contiguous(), gpu["actions"][idx], gpu["old_lp"][idx], gpu["adv"][idx],
        gpu["ret"][idx], v2(obs_b).squeeze(1).contiguous())
    loss.backward()
    for a, b in zip(list(p1.parameters()) + list(v1.parameters()),
                    list(p2.parameters()) + list(v2.parameters())):
        assert_grad_close(a.grad, b.grad)


@pytest.mark.parametrize("capturable", [False, True])
@pytest.mark.parametrize("max_norm", [0.5, 1e6])
def test_mlp_step_matches_grads_then_clipped_adam(dev, capturable, max_norm):
    """ppo_mlp_cat_step_f32 (gradients + clip + Adam in two or three launches) against
    ppo_mlp_cat_grads followed by ClippedAdam.step(), over four steps: the
    gradients are the same; the clip norm is summed from 64-element pieces
    instead of 1024-element ones (fp64), so parameters, moments and norms
    agree within 2e-6 relative."""
    pol, val, cpu, gpu = _case(dev, 512, 4, 64, 2, "tanh", seed=21)
    nets = [(copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)) for _ in range(2)]
    opts = [ppo_amd.ClippedAdam(list(p.parameters()) + list(v.parameters()), lr=1e-3,
                                max_grad_norm=max_norm, capturable=capturable)
            for p, v in nets]
    args = (gpu["obs"], gpu["actions"], gpu["old_lp"], gpu["adv"], gpu["ret"])
    g = torch.Generator().manual_seed(22)
    for step in range(4):
        idx = torch.randperm(512, generator=g)[:256].to(dev)
        s1, n1 = ppo_amd.ppo_mlp_cat_step(nets[0][0], nets[0][1], opts[0], *args, index=idx)
        s2 = ppo_amd.ppo_mlp_cat_grads(nets[1][0], nets[1][1], *args, index=idx)
        n2 = opts[1].step()
        assert n1.item() == pytest.approx(n2.item(), rel=2e-6)
        for k in s2:
            assert torch.equal(s1[k], s2[k]), k
        for a, b in zip(opts[0].params, opts[1].params):
            torch.testing.assert_close(a.grad, b.grad, rtol=2e-6, atol=1e-9)
            torch.testing.assert_close(a.detach(), b.detach(), rtol=2e-6, atol=1e-7)
    for a, b in zip(opts[0].exp_avg + opts[0].exp_avg_sq, opts[1].exp_avg + opts[1].exp_avg_sq):
        torch.testing.assert_close(a, b, rtol=2e-6, atol=1e-10)
    assert opts[0].step_count() == opts[1].step_count() == 4


@pytest.mark.parametrize("capturable", [False, True])
@pytest.mark.parametrize("max_norm,n,B", [(0.5, 512, 256), (1e6, 512, 256), (0.5, 8192, 4096)])
def test_mlp_step_one_launch_matches_two(dev, monkeypatch, capturable, max_norm, n, B):
    """ppo_mlp_cat_step_f32 sums the gradient partials and applies clip + Adam
    in one launch when its grid is resident (an in-kernel barrier between the
    sums of squares and the update); PPO_AMD_MLP_FUSED_ADAM=0 keeps the
    reduction and the update as two launches.  Both must give bit-identical
    gradients, parameters, moments, norms, loss scalars and step counts, over
    four steps (B = 4096 takes the 1024-thread reduction geometry)."""
    pol, val, cpu, gpu = _case(dev, n, 4, 64, 2, "tanh", seed=41)
    nets = [(copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)) for _ in range(2)]
    opts = [ppo_amd.ClippedAdam(list(p.parameters()) + list(v.parameters()), lr=1e-3,
                                max_grad_norm=max_norm, capturable=capturable)
            for p, v in nets]
    args = (gpu["obs"], gpu["actions"], gpu["old_lp"], gpu["adv"], gpu["ret"])
    g = torch.Generator().manual_seed(42)
    for step in range(4):
        idx = torch.randperm(n, generator=g)[:B].to(dev)
        print(f"mlp step fused-vs-two n={n} B={B} step={step} capturable={capturable}",
              flush=True)
        monkeypatch.delenv("PPO_AMD_MLP_FUSED_ADAM", raising=False)
        s1, n1 = ppo_amd.ppo_mlp_cat_step(nets[0][0], nets[0][1], opts[0], *args, index=idx)
        monkeypatch.setenv("PPO_AMD_MLP_FUSED_ADAM", "0")
        s2, n2 = ppo_amd.ppo_mlp_cat_step(nets[1][0], nets[1][1], opts[1], *args, index=idx)
        torch.cuda.synchronize(dev)
        assert torch.equal(n1, n2)
        for k in s2:
            assert torch.equal(s1[k], s2[k]), k
        for a, b in zip(opts[0].params, opts[1].params):
            assert torch.equal(a.grad, b.grad)
            assert torch.equal(a.detach(), b.detach())
    for a, b in zip(opts[0].exp_avg + opts[0].exp_avg_sq, opts[1].exp_avg + opts[1].exp_avg_sq):
        assert torch.equal(a, b)
    assert opts[0].step_count() == opts[1].step_count() == 4


def test_mlp_step_rejects_foreign_optimizer(dev):
    pol, val, cpu, gpu = _case(dev, 64, 4, 32, 2, "tanh", seed=23)
    p, v = pol.to(dev), val.to(dev)
    opt = ppo_amd.ClippedAdam(list(v.parameters()) + list(p.parameters()))  # wrong order
    with pytest.raises(ValueError):
        ppo_amd.ppo_mlp_cat_step(p, v, opt, gpu["obs"], gpu["actions"], gpu["old_lp"],
                                 gpu["adv"], gpu["ret"])


def test_mlp_grads_deterministic(dev):
    pol, val, cpu, gpu = _case(dev, 2048, 4, 128, 2, "relu", seed=11)
    idx = torch.randperm(2048, generator=torch.Generator().manual_seed(12))[:1000].to(dev)
    pd, vd = pol.to(dev), val.to(dev)
    args = (gpu["obs"], gpu["actions"], gpu["old_lp"], gpu["adv"], gpu["ret"])
    ppo_amd.ppo_mlp_cat_grads(pd, vd, *args, index=idx)
    first = [p.grad.clone() for p in list(pd.parameters()) + list(vd.parameters())]
    ppo_amd.ppo_mlp_cat_grads(pd, vd, *args, index=idx)
    for a, p in zip(first, list(pd.parameters()) + list(vd.parameters())):
        assert torch.equal(a, p.grad)


def test_mlp_fusable_rejects_other_networks(dev):
    a = MLP(4, 64, 2, "tanh").to(dev)
    assert ppo_amd.mlp_fusable(a, MLP(4, 64, 1, "tanh").to(dev))
    assert not ppo_amd.mlp_fusable(a, MLP(4, 64, 1, "relu").to(dev))      # activations differ
    assert not ppo_amd.mlp_fusable(a, MLP(4, 32, 1, "tanh").to(dev))      # hidden differs
    assert not ppo_amd.mlp_fusable(MLP(4, 48, 2).to(dev), MLP(4, 48, 1).to(dev))  # H = 48
    assert not ppo_amd.mlp_fusable(MLP(4, 64, 33).to(dev), MLP(4, 64, 1).to(dev))  # A > 32
    assert not ppo_amd.mlp_fusable(MLP(4, 64, 2), MLP(4, 64, 1))          # on the CPU
    with pytest.raises(ValueError):
        ppo_amd.ppo_mlp_cat_grads(MLP(4, 48, 2).to(dev), MLP(4, 48, 1).to(dev),
                                  torch.zeros(4, 4, device=dev),
                                  torch.zeros(4, dtype=torch.int32, device=dev),
                                  *(torch.zeros(4, device=dev) for _ in range(3)))


@pytest.mark.parametrize("graphs", [False, True])
def test_vecppo_fused_mlp_matches_unfused(dev, graphs):
    """VecPPO with the fused MLP minibatch kernel against VecPPO with torch's
    MLPs + the fused loss op, same rollout and permutations: parameters after
    two updates (4 epochs x 5 minibatches each) agree to 1e-5 (Adam moves each
    parameter by at most ~lr = 3e-4 per step)."""
    T, N = 40, 8
    torch.manual_seed(21)
    policy, value = MLP(4, 64, 2, "tanh").to(dev), MLP(4, 64, 1, "tanh").to(dev)
    made = []
    for fused in (True, False):
        made.append(ppo_amd.VecPPO(copy.deepcopy(policy), copy.deepcopy(value), batch_size=64,
                                   generator=torch.Generator().manual_seed(2), graphs=graphs,
                                   fused_mlp=fused))
    assert made[0].fused_mlp and not made[1].fused_mlp
    g = torch.Generator().manual_seed(22)
    buf = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    for _ in range(T):
        buf.add(torch.randn(N, 4, generator=g).to(dev),
                torch.randint(0, 2, (N,), generator=g, dtype=torch.int32).to(dev),
                torch.ones(N).to(dev), (torch.rand(N, generator=g) < 0.02).to(torch.uint8).to(dev),
                torch.randn(N, generator=g).to(dev), (torch.randn(N, generator=g) - 0.7).to(dev))
    buf.finish(None)
    for _ in range(2):
        s_f = made[0].update(buf)
        s_u = made[1].update(buf)
    torch.cuda.synchronize()
    for a, b in zip(made[0].parameters, made[1].parameters):
        torch.testing.assert_close(a.detach(), b.detach(), rtol=0, atol=1e-5)
    for k in ("loss", "policy", "value", "entropy"):
        torch.testing.assert_close(s_f[k], s_u[k], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("H,A,act", [(64, 2, "tanh"), (128, 5, "relu"), (32, 18, "tanh")])
def test_mlp_act_matches_torch_forward_and_sampler(dev, H, A, act):
    """ppo_mlp_act_cat_f32 (both forwards + the inverse-CDF draw in one
    launch) against torch's MLP forwards + ppo_sample_cat_f32 at the same
    uniforms: values and log-probs within 1e-5, actions equal except rows
    whose uniform lies within 1e-5 of a CDF boundary (the two forwards round
    differently), observations copied exactly."""
    torch.manual_seed(H + A)
    N, D = 1000, 6
    pol, val = MLP(D, H, A, act).to(dev), MLP(D, H, 1, act).to(dev)
    obs = torch.randn(N, D, device=dev)
    u = torch.rand(N, device=dev)
    obs_out = torch.empty(N, D, device=dev)
    a1, lp1, v1 = ppo_amd.mlp_act_categorical(pol, val, obs, u, observations_out=obs_out)
    with torch.no_grad():
        logits = pol(obs)
        v2 = val(obs).squeeze(1)
    a2, lp2 = ppo_amd.sample_categorical(logits.contiguous(), u)
    _, _, margin = ref.sample_categorical_reference(logits.cpu().double().numpy(),
                                                    u.cpu().double().numpy())
    clear = torch.from_numpy(margin > 1e-5)
    assert clear.float().mean() > 0.95
    assert torch.equal(a1.cpu()[clear], a2.cpu()[clear])
    torch.testing.assert_close(lp1.cpu()[clear], lp2.cpu()[clear], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(v1, v2, rtol=1e-5, atol=1e-5)
    assert torch.equal(obs_out, obs)
