"""GPU parity of batched action selection (ppo_sample_cat_f32 /
ppo_sample_gauss_f32, PPOAgent.select_action at ppo.py:65-79 batched over
envs) against oracle.sample_categorical_reference and torch.distributions.

Tolerances: the sampled action is an integer and must match the fp64
inverse-CDF oracle exactly, except on rows whose uniform lies within 1e-5 of
a CDF boundary (fp32 softmax sums may round across it); log-probs within
2e-6 absolute of fp64; Gaussian actions within 1e-6 relative (exp of log_std
on the device vs in torch), log-probs within 2e-5 absolute; values copied
bit-exactly.
"""

import numpy as np
import pytest
import torch

import ppo_amd
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,A", [(1, 2), (8, 2), (300, 18), (4096, 5), (1000, 64), (257, 65),
                                 (64, 300), (3, 1)])
def test_sample_categorical_matches_inverse_cdf_oracle(dev, N, A):
    g = torch.Generator().manual_seed(N * 1000 + A)
    logits = torch.randn(N, A, generator=g) * 2.0
    u = torch.rand(N, generator=g)
    vals = torch.randn(N, generator=g)
    vout = torch.full((N,), float("nan"))
    acts, logp = ppo_amd.sample_categorical(logits.to(dev), u.to(dev), values=vals.to(dev),
                                            values_out=vout.to(dev))
    a_ref, lp_ref, margin = ref.sample_categorical_reference(logits.numpy(), u.numpy())
    got = acts.cpu().numpy()
    assert acts.dtype == torch.int32 and got.min() >= 0 and got.max() < A
    ok = margin > 1e-5
    assert np.array_equal(got[ok], a_ref[ok])
    # log-prob of the action actually drawn, against fp64 log_softmax
    z = logits.double()
    want = (z - torch.logsumexp(z, 1, keepdim=True)).gather(1, acts.cpu().long()[:, None])
    np.testing.assert_allclose(logp.cpu().numpy(), want.squeeze(1).numpy(), rtol=0, atol=2e-6)


def test_sample_categorical_values_copied_and_rows_written_in_place(dev):
    N, A, T = 37, 4, 3
    logits = torch.randn(N, A, device=dev)
    vals = torch.randn(N, device=dev)
    acts_buf = torch.full((T, N), -7, dtype=torch.int32, device=dev)
    lp_buf = torch.zeros(T, N, device=dev)
    v_buf = torch.zeros(T, N, device=dev)
    ppo_amd.sample_categorical(logits, torch.rand(N, device=dev), values=vals,
                               actions_out=acts_buf[1], log_probs_out=lp_buf[1],
                               values_out=v_buf[1])
    assert torch.equal(v_buf[1], vals)
    assert (acts_buf[0] == -7).all() and (acts_buf[2] == -7).all()
    assert ((acts_buf[1] >= 0) & (acts_buf[1] < A)).all()


def test_sample_categorical_frequencies(dev):
    N, A = 400_000, 6
    g = torch.Generator(device=dev).manual_seed(5)
    z = torch.randn(A) * 1.3
    logits = z[None].repeat(N, 1).to(dev)
    acts, _ = ppo_amd.sample_categorical(logits, generator=g)
    freq = torch.bincount(acts.long().cpu(), minlength=A).double() / N
    p = torch.softmax(z.double(), 0)
    assert torch.all((freq - p).abs() < 5 * torch.sqrt(p * (1 - p) / N))


@pytest.mark.parametrize("N,D", [(1, 1), (100, 6), (4097, 3), (50, 24)])
def test_sample_gaussian_matches_torch_normal(dev, N, D):
    g = torch.Generator().manual_seed(N + D)
    mu = torch.randn(N, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0
    eps = torch.randn(N, D, generator=g)
    vals = torch.randn(N, generator=g)
    acts, logp = ppo_amd.sample_gaussian(mu.to(dev), log_std.to(dev), eps.to(dev),
                                         values=vals.to(dev),
                                         values_out=torch.empty(N, device=dev))
    want = mu + log_std.exp() * eps
    torch.testing.assert_close(acts.cpu(), want, rtol=1e-6, atol=1e-6)
    dist = torch.distributions.Normal(mu.double(), log_std.double().exp())
    want_lp = dist.log_prob(acts.cpu().double()).sum(-1)
    np.testing.assert_allclose(logp.cpu().numpy(), want_lp.numpy(), rtol=0, atol=2e-5)


@pytest.mark.parametrize("fused_mlp", [False, True])
def test_vecppo_act_fills_buffer_rows(dev, fused_mlp):
    """VecPPO.act writes row t of the buffer: torch's MLPs + the sampling
    kernel (exact against torch's forward), or the fused forward + sampling
    kernel (MFMA forward: values and log-probs within 1e-5)."""
    from ppo_amd.agent import MLP

    torch.manual_seed(2)
    T, N = 4, 16
    policy, value = MLP(4, 32, 3, "tanh").to(dev), MLP(4, 32, 1, "tanh").to(dev)
    vec = ppo_amd.VecPPO(policy, value, fused_mlp=fused_mlp)
    tol = 1e-5 if fused_mlp else 0.0
    buf = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
    g = torch.Generator(device=dev).manual_seed(11)
    for t in range(T):
        obs = torch.randn(N, 4, device=dev)
        acts, logp, vals = vec.act(obs, buffer=buf, generator=g)
        assert acts.data_ptr() == buf.actions[t].data_ptr()
        with torch.no_grad():
            z = policy(obs)
            want_v = value(obs).squeeze(1)
        assert torch.equal(buf.observations[t], obs)
        torch.testing.assert_close(buf.values[t], want_v, rtol=0, atol=tol)
        want_lp = torch.log_softmax(z, 1).gather(1, buf.actions[t].long()[:, None]).squeeze(1)
        torch.testing.assert_close(buf.log_probs[t], want_lp, rtol=0, atol=2e-6 + tol)
        buf.add_outcome(torch.ones(N, device=dev), torch.zeros(N, dtype=torch.uint8, device=dev))
    assert buf.step == T
    with pytest.raises(IndexError):
        vec.act(torch.randn(N, 4, device=dev), buffer=buf)
    # the filled buffer feeds the update directly
    buf.finish(None)
    stats = vec.update(buf)
    assert torch.isfinite(stats["loss"]).item()
