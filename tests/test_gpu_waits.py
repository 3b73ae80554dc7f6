"""Bounded in-kernel waits that give up fail loudly.

Four launches hold workgroups that wait for one another: the resident GAE
pass, the in-kernel finish of the Gaussian loss and of the categorical loss,
and the fused clip + Adam of ppo_mlp_cat_step.  The give-up is forced from the host with a poll limit of
zero (ppo_set_wait_limit), so every wait gives up at once and every kernel
still exits normally.  Then:
  - ppo_wait_status / ops.check_waits raise PPO_ERR_WAIT_TIMEOUT, once (the
    status word is cleared by the check);
  - GAE outputs are NaN; the Gaussian loss scalars formed from the collected
    sums and dlog_std are NaN;
  - the fused Adam step leaves parameters, moments, gradients and the step
    counter unchanged bit for bit, and its norm output is NaN;
  - with the default limit restored, the same calls give the results of the
    launches without in-kernel waits, bit for bit.
"""

import copy

import numpy as np
import pytest
import torch

import ppo_amd
from ppo_amd import _lib, ops
from ppo_amd.agent import MLP, PPOConfig
from ppo_amd.rollout import RolloutBuffer, VecPPO
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu


@pytest.fixture
def giveup(dev):
    """Clears any earlier status, yields a context that sets the limit to
    zero, and restores the default limit afterwards."""
    ops.check_waits(dev)

    class _Ctx:
        def __enter__(self):
            ops.set_wait_limit(0)

        def __exit__(self, *exc):
            ops.set_wait_limit(None)
            return False

    try:
        yield _Ctx()
    finally:
        ops.set_wait_limit(None)


def _expect_timeout(dev):
    with pytest.raises(_lib.PPOLibraryError) as ei:
        ops.check_waits(dev)
    assert ei.value.code == _lib.PPO_ERR_WAIT_TIMEOUT
    ops.check_waits(dev)  # cleared by the check that reported it


def _rollout(T, N, p_done, seed):
    g = torch.Generator().manual_seed(seed)
    r = torch.randn(T, N, generator=g)
    v = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < p_done).to(torch.uint8)
    lv = torch.randn(N, generator=g)
    return r, v, d, lv


@pytest.mark.parametrize("T,N,norm,gamma", [
    (2048, 4096, True, 0.99),       # configuration 2's shape
    (2048, 4096, False, 0.99),
    (1 << 20, 16, False, 0.999),    # configuration 3's shape (two rounds)
])
def test_gae_resident_giveup_writes_nan_and_reports(dev, giveup, T, N, norm, gamma):
    lib = _lib.load()
    assert lib.ppo_gae_route(T, N, int(norm), 1) == 1, "shape must take the resident pass"
    print(f"waits gae T={T} N={N} norm={norm}", flush=True)
    r, v, d, lv = (x.to(dev) for x in _rollout(T, N, 0.01 if N > 16 else 0.001, 5))
    run = (lambda: ops.gae_normalize(r, v, d, lv, gamma, 0.95)) if norm else (
        lambda: ops.gae(r, v, d, lv, gamma, 0.95))
    good = [x.clone() for x in run()]
    ops.check_waits(dev)
    with giveup:
        bad = run()
        torch.cuda.synchronize(dev)
    for x in bad:
        assert bool(torch.isnan(x).all()), "every output element of a failed call is NaN"
    _expect_timeout(dev)
    again = run()
    ops.check_waits(dev)
    for a, b in zip(good, again):
        assert torch.equal(a, b)
    # and the results are the oracle's (bit-exact advantages)
    if not norm and N > 16:
        adv_ref, _ = ref.gae_numpy(r.cpu().numpy(), v.cpu().numpy(), d.cpu().numpy(),
                                lv.cpu().numpy(), gamma, 0.95)
        assert np.array_equal(again[0].cpu().numpy(), adv_ref.astype(np.float32))


def _gauss(dev, B, D, seed):
    g = torch.Generator().manual_seed(seed)
    mu = torch.randn(B, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0
    acts = mu + 0.05 * torch.randn(B, D, generator=g) + log_std.exp() * torch.randn(
        B, D, generator=g)
    old_lp = torch.distributions.Normal(mu, log_std.exp()).log_prob(acts).sum(-1) + 0.01
    adv, ret, val, old_v = (torch.randn(B, generator=g) for _ in range(4))
    return [x.to(dev) for x in (mu, log_std, acts, old_lp, adv, ret, val, old_v)]


@pytest.mark.parametrize("B,D", [(8_388_608, 6), (2_097_152, 6), (100_003, 3), (4096, 17),
                                 (5_000_003, 8)])
def test_gauss_finish_giveup_and_launch_route(dev, giveup, monkeypatch, B, D):
    print(f"waits gauss B={B} D={D}", flush=True)
    args = _gauss(dev, B, D, 9)
    monkeypatch.delenv("PPO_AMD_GAUSS_FINISH", raising=False)
    good = [x.clone() for x in ops.ppo_loss_gaussian_fused(*args, 0.2, 0.2, 0.5, 0.01)]
    # the finish as a launch of its own (no in-kernel wait): bit-identical
    monkeypatch.setenv("PPO_AMD_GAUSS_FINISH", "0")
    sep = ops.ppo_loss_gaussian_fused(*args, 0.2, 0.2, 0.5, 0.01)
    for a, b in zip(good, sep):
        assert torch.equal(a, b)
    ops.check_waits(dev)
    for route in ("1", "0"):
        monkeypatch.setenv("PPO_AMD_GAUSS_FINISH", route)
        with giveup:
            scalars, dmu, dls, dv = ops.ppo_loss_gaussian_fused(*args, 0.2, 0.2, 0.5, 0.01)
            torch.cuda.synchronize(dev)
        assert torch.equal(dmu, good[1]) and torch.equal(dv, good[3])  # per-row outputs
        if route == "0":
            # the finish as a launch of its own waits for nothing
            assert torch.equal(scalars, good[0]) and torch.equal(dls, good[2])
            ops.check_waits(dev)
            continue
        # every scalar formed from the collected sums is NaN; the entropy of a
        # state-independent Normal comes from log_std alone and stays valid
        summed = [k for k in range(6) if k != 3]
        assert bool(torch.isnan(scalars[summed]).all()) and bool(torch.isnan(dls).all()), route
        assert torch.equal(scalars[3], good[0][3])
        _expect_timeout(dev)
    monkeypatch.delenv("PPO_AMD_GAUSS_FINISH", raising=False)
    again = ops.ppo_loss_gaussian_fused(*args, 0.2, 0.2, 0.5, 0.01)
    ops.check_waits(dev)
    for a, b in zip(good, again):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,A", [(8_388_608, 18), (1_048_576, 18), (70_001, 5), (4096, 2),
                                 (5_000_001, 8), (3000, 24)])
def test_categorical_finish_giveup_and_launch_route(dev, giveup, monkeypatch, B, A):
    """The categorical loss finishes in-kernel (workgroup 0 collects the
    tagged partials; on the wave-tile kernels it takes no tiles itself);
    PPO_AMD_CAT_FINISH=0 selects the finaliser launch instead.  Both give the same results bit for bit; a give-up
    leaves NaN scalars, intact gradients and the status raised."""
    print(f"waits cat B={B} A={A}", flush=True)
    g = torch.Generator().manual_seed(B)
    logits = torch.randn(B, A, generator=g)
    acts = torch.randint(0, A, (B,), generator=g, dtype=torch.int32)
    rows = [torch.randn(B, generator=g) for _ in range(5)]
    args = [x.to(dev) for x in [logits, acts] + rows]
    monkeypatch.delenv("PPO_AMD_CAT_FINISH", raising=False)
    good = [x.clone() for x in ops.ppo_loss_discrete_fused(*args, 0.2, 0.2, 0.5, 0.01)]
    monkeypatch.setenv("PPO_AMD_CAT_FINISH", "0")
    sep = ops.ppo_loss_discrete_fused(*args, 0.2, 0.2, 0.5, 0.01)
    for a, b in zip(good, sep):
        assert torch.equal(a, b)
    monkeypatch.delenv("PPO_AMD_CAT_FINISH", raising=False)
    ops.check_waits(dev)
    # the wave-tile forms (A % 4 != 0, A <= 20) finish in-kernel at every B,
    # the other forms up to 2^22 rows; above that the finaliser launch waits
    # for nothing
    in_kernel = (A % 4 != 0 and A <= 20) or B <= (1 << 22)
    with giveup:
        scalars, dlogits, dv = ops.ppo_loss_discrete_fused(*args, 0.2, 0.2, 0.5, 0.01)
        torch.cuda.synchronize(dev)
    assert torch.equal(dlogits, good[1]) and torch.equal(dv, good[2])
    if in_kernel:
        assert bool(torch.isnan(scalars).all())
        _expect_timeout(dev)
    else:
        assert torch.equal(scalars, good[0])
        ops.check_waits(dev)
    again = ops.ppo_loss_discrete_fused(*args, 0.2, 0.2, 0.5, 0.01)
    ops.check_waits(dev)
    for a, b in zip(good, again):
        assert torch.equal(a, b)


def _mlp_case(dev, n, seed):
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    pol, val = MLP(4, 64, 2, "tanh"), MLP(4, 64, 1, "tanh")
    obs = torch.randn(n, 4, generator=g)
    acts = torch.randint(0, 2, (n,), generator=g, dtype=torch.int32)
    old_lp = -0.7 + 0.1 * torch.randn(n, generator=g)
    adv, ret = torch.randn(n, generator=g), torch.randn(n, generator=g)
    return pol, val, [x.to(dev) for x in (obs, acts, old_lp, adv, ret)]


@pytest.mark.parametrize("capturable", [False, True])
@pytest.mark.parametrize("n,B", [(512, 256), (8192, 4096)])
def test_fused_adam_giveup_leaves_parameters(dev, giveup, monkeypatch, capturable, n, B):
    print(f"waits mlp adam n={n} B={B} capturable={capturable}", flush=True)
    monkeypatch.delenv("PPO_AMD_MLP_FUSED_ADAM", raising=False)
    pol, val, args = _mlp_case(dev, n, 31)
    nets = [(copy.deepcopy(pol).to(dev), copy.deepcopy(val).to(dev)) for _ in range(2)]
    opts = [ppo_amd.ClippedAdam(list(p.parameters()) + list(v.parameters()), lr=1e-3,
                                max_grad_norm=0.5, capturable=capturable) for p, v in nets]
    g = torch.Generator().manual_seed(32)
    idx = torch.randperm(n, generator=g)[:B].to(dev)
    # one good step on both, so moments and grads are non-trivial
    for (p, v), o in zip(nets, opts):
        ops.ppo_mlp_cat_step(p, v, o, *args, index=idx)
    ops.check_waits(dev)
    before = [t.clone() for t in opts[0].params + opts[0].exp_avg + opts[0].exp_avg_sq]
    grads = [t.grad.clone() for t in opts[0].params]
    count = opts[0].step_t.clone() if capturable else None
    idx2 = torch.randperm(n, generator=g)[:B].to(dev)
    with giveup:
        _, norm = ops.ppo_mlp_cat_step(nets[0][0], nets[0][1], opts[0], *args, index=idx2)
        torch.cuda.synchronize(dev)
    after = opts[0].params + opts[0].exp_avg + opts[0].exp_avg_sq
    for a, b in zip(before, after):
        assert torch.equal(a, b.detach()), "a failed wait must not write parameters or moments"
    for a, p in zip(grads, opts[0].params):
        assert torch.equal(a, p.grad)
    if capturable:
        assert torch.equal(count, opts[0].step_t)
    assert bool(torch.isnan(norm))
    _expect_timeout(dev)
    # restore the state the failed step left logically untouched, then the
    # fused step equals the two-launch step bit for bit
    if not capturable:
        opts[0].steps = list(opts[1].steps)
    ops.ppo_mlp_cat_step(nets[0][0], nets[0][1], opts[0], *args, index=idx2)
    monkeypatch.setenv("PPO_AMD_MLP_FUSED_ADAM", "0")
    ops.ppo_mlp_cat_step(nets[1][0], nets[1][1], opts[1], *args, index=idx2)
    ops.check_waits(dev)
    for a, b in zip(opts[0].params + opts[0].exp_avg + opts[0].exp_avg_sq,
                    opts[1].params + opts[1].exp_avg + opts[1].exp_avg_sq):
        assert torch.equal(a.detach(), b.detach())


@pytest.mark.parametrize("mode", ["deferred", "sync"])
def test_vecppo_update_raises_on_giveup(dev, giveup, mode):
    """VecPPO.update checks the wait status once per update: "sync" at the
    end of the update that gave up, "deferred" at the end of the next update
    (or at flush_waits)."""
    torch.manual_seed(3)
    T, N = 64, 64
    pol, val = MLP(4, 64, 2, "tanh").to(dev), MLP(4, 64, 1, "tanh").to(dev)
    agent = VecPPO(pol, val, PPOConfig(), batch_size=1024, check_waits=mode)
    assert agent.fused_mlp
    buf = RolloutBuffer(T, N, (4,), device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    for _ in range(T):
        obs = torch.rand(N, 4, device=dev, generator=g) - 0.5
        agent.act(obs, buf)
        buf.add_outcome(torch.ones(N, device=dev),
                        (torch.rand(N, device=dev, generator=g) < 0.02).to(torch.uint8))
    buf.finish()
    before = [p.detach().clone() for p in agent.parameters]
    with giveup:
        if mode == "deferred":
            agent.update(buf)  # (reported by the next check)
            with pytest.raises(_lib.PPOLibraryError) as ei:
                agent.flush_waits()
        else:
            with pytest.raises(_lib.PPOLibraryError) as ei:
                agent.update(buf)
    assert ei.value.code == _lib.PPO_ERR_WAIT_TIMEOUT
    for a, b in zip(before, agent.parameters):
        assert torch.equal(a, b.detach())  # every minibatch's Adam step gave up
    ops.check_waits(dev)
    agent.flush_waits()
    # a clean update after the reset, then a deferred report of nothing
    agent.update(buf)
    agent.update(buf)
    agent.flush_waits()
    assert any(not torch.equal(a, b.detach()) for a, b in zip(before, agent.parameters))


def test_wait_poller_reports_previous_iteration(dev, giveup):
    """WaitPoller.check reports a give-up of the previous iteration, clears
    the workspaces, and then runs clean."""
    poller = ops.WaitPoller()
    r, v, d, lv = (x.to(dev) for x in _rollout(2048, 4096, 0.01, 5))
    good = [x.clone() for x in ops.gae_normalize(r, v, d, lv, 0.99, 0.95)]
    poller.check(dev)
    with giveup:
        ops.gae_normalize(r, v, d, lv, 0.99, 0.95)
    poller.check(dev)  # takes the give-up, reports the clean iteration before
    ops.gae_normalize(r, v, d, lv, 0.99, 0.95)  # (invalid until the report: may be stale)
    with pytest.raises(_lib.PPOLibraryError) as ei:
        poller.check(dev)
    assert ei.value.code == _lib.PPO_ERR_WAIT_TIMEOUT
    again = ops.gae_normalize(r, v, d, lv, 0.99, 0.95)
    poller.check(dev)
    poller.flush(dev)
    for a, b in zip(good, again):
        assert torch.equal(a, b)
