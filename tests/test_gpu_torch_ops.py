"""torch.ops.ppo_amd.* on the GPU: each operator equals the ppo_amd.ops
function it wraps bit for bit, passes torch.library.opcheck (schema, fake
tensor, autograd registration, AOT dispatch), and a compiled PPO update step
(torch.compile, fullgraph, through the fake implementations) gives the eager
step's results and gradients."""

import pytest
import torch

import ppo_amd
from ppo_amd import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _rollout(dev, T, N, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    r = torch.randn(T, N, device=dev, generator=g)
    v = torch.randn(T, N, device=dev, generator=g)
    d = (torch.rand(T, N, device=dev, generator=g) < 0.05).to(torch.uint8)
    lv = torch.randn(N, device=dev, generator=g)
    return r, v, d, lv


def _cat(dev, B, A, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    logits = torch.randn(B, A, device=dev, generator=g)
    act = torch.randint(0, A, (B,), device=dev, generator=g)
    old_lp = torch.log_softmax(logits, -1).gather(1, act[:, None]).squeeze(1)
    old_lp = old_lp + 0.1 * torch.randn(B, device=dev, generator=g)
    adv, ret, val, old_v = (torch.randn(B, device=dev, generator=g) for _ in range(4))
    return logits, act, old_lp, adv, ret, val, old_v


def test_ops_equal_functions(dev):
    print("torch ops vs ops functions", flush=True)
    r, v, d, lv = _rollout(dev, 256, 64, 1)
    for got, want in zip(torch.ops.ppo_amd.gae(r, v, d, lv, 0.99, 0.95),
                         ops.gae(r, v, d, lv, 0.99, 0.95)):
        assert torch.equal(got, want)
    for got, want in zip(torch.ops.ppo_amd.gae_normalize(r, v, d, None, 0.99, 0.95, 1e-8),
                         ops.gae_normalize(r, v, d, None, 0.99, 0.95, 1e-8, return_stats=True)):
        assert torch.equal(got, want)
    assert torch.equal(torch.ops.ppo_amd.normalize_advantages(r, 1e-8),
                       ops.normalize_advantages(r, 1e-8))
    x = _cat(dev, 1000, 6, 2)
    for got, want in zip(torch.ops.ppo_amd.ppo_loss_discrete(*x, 0.2, 0.2, 0.5, 0.01),
                         ops.ppo_loss_discrete_fused(*x, 0.2, 0.2, 0.5, 0.01)):
        assert torch.equal(got, want)


def _opcheck_cases(dev):
    r, v, d, lv = _rollout(dev, 64, 16, 3)
    logits, act, old_lp, adv, ret, val, old_v = _cat(dev, 300, 4, 4)
    g = torch.Generator(device=dev).manual_seed(5)
    mu = torch.randn(300, 3, device=dev, generator=g)
    ls = torch.rand(3, device=dev, generator=g) - 1.0
    acts = mu + ls.exp() * torch.randn(300, 3, device=dev, generator=g)
    glp = torch.distributions.Normal(mu, ls.exp()).log_prob(acts).sum(-1)
    return [
        (torch.ops.ppo_amd.gae.default, (r, v, d, lv, 0.99, 0.95)),
        (torch.ops.ppo_amd.gae_normalize.default, (r, v, d, None, 0.99, 0.95, 1e-8)),
        (torch.ops.ppo_amd.normalize_advantages.default, (adv, 1e-8)),
        (torch.ops.ppo_amd.ppo_loss_discrete.default,
         (logits.requires_grad_(), act, old_lp, adv, ret, val.clone().requires_grad_(), old_v,
          0.2, 0.2, 0.5, 0.01)),
        (torch.ops.ppo_amd.ppo_loss_gaussian.default,
         (mu.requires_grad_(), ls.requires_grad_(), acts, glp, adv, ret,
          val.clone().requires_grad_(), None, 0.2, None, 0.5, 0.01)),
    ]


@pytest.mark.parametrize("case", range(5))
def test_opcheck(dev, case):
    op, args = _opcheck_cases(dev)[case]
    print(f"opcheck {op}", flush=True)
    torch.library.opcheck(op, args)


def test_compiled_step_matches_eager(dev):
    """GAE + normalisation + the categorical loss through a linear policy and
    value head, compiled whole (fullgraph, aot_eager: the operators trace via
    their fake implementations, the backward via their registered autograd),
    against the same step run eagerly."""
    print("torch.compile step", flush=True)
    T, N, obs, A = 128, 32, 8, 5
    r, v, d, lv = _rollout(dev, T, N, 6)
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(T * N, obs, device=dev, generator=g)
    act = torch.randint(0, A, (T * N,), device=dev, generator=g)
    old_lp = torch.randn(T * N, device=dev, generator=g) - 2.0

    def step(wp, wv):
        adv, ret, adv_n, _ = torch.ops.ppo_amd.gae_normalize(r, v, d, lv, 0.99, 0.95, 1e-8)
        logits = x @ wp
        values = (x @ wv).squeeze(1)
        scalars, _, _ = torch.ops.ppo_amd.ppo_loss_discrete(
            logits, act, old_lp, adv_n.reshape(-1), ret.reshape(-1), values, None,
            0.2, None, 0.5, 0.01)
        return scalars

    torch._dynamo.reset()
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    results = []
    for fn in (step, compiled):
        wp = torch.randn(obs, A, device=dev, generator=torch.Generator(device=dev).manual_seed(8))
        wv = torch.randn(obs, 1, device=dev, generator=torch.Generator(device=dev).manual_seed(9))
        wp.requires_grad_()
        wv.requires_grad_()
        s = fn(wp, wv)
        s[0].backward()  # (through the registered backward, traced by AOT autograd)
        results.append((s.detach().clone(), wp.grad.clone(), wv.grad.clone()))
    (s0, gp0, gv0), (s1, gp1, gv1) = results
    assert torch.isfinite(s0).all()
    torch.testing.assert_close(s1, s0, rtol=0, atol=0)
    torch.testing.assert_close(gp1, gp0, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(gv1, gv0, rtol=1e-6, atol=1e-7)
