"""GPU parity of advantage normalisation (ppo.py:126-127) against the
reference's torch-CPU expression, and of the fused GAE+normalise path.

Tolerance: rel 1e-5 (the benchmark's stated bar) with atol 1e-6 for elements near the mean.
The kernel's mean/std are fp64 sums rounded to fp32; torch's are fp32
reductions, so the two can differ by a few fp32 ulps.
"""

import numpy as np
import pytest
import torch

import ppo_amd
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _c_oracle():
    ref.build_c()


@pytest.mark.parametrize("n", [2, 3, 4, 5, 255, 1024, 4099, 1_000_003])
def test_normalize_matches_reference(dev, n):
    g = torch.Generator().manual_seed(n)
    a = torch.randn(n, generator=g) * 2.5 + 0.7
    print(f"normalize n={n}", flush=True)
    out = ppo_amd.normalize_advantages(a.to(dev))
    expect = ref.normalize_reference(a)
    torch.testing.assert_close(out.cpu(), expect, rtol=1e-5, atol=1e-6)


def test_normalize_single_element_is_identity(dev):
    a = torch.tensor([-4.5], device=dev)
    out = ppo_amd.normalize_advantages(a)
    assert out.item() == -4.5


@pytest.mark.parametrize("n", [2, 1000, 1_048_579])
def test_normalize_constant_advantages(dev, n):
    """Equal advantages: std 0, so (adv - mean) / (0 + eps) is exactly zero in
    the reference's expression and here (no NaN from the variance)."""
    a = torch.full((n,), 3.25)
    out = ppo_amd.normalize_advantages(a.to(dev)).cpu()
    expect = ref.normalize_reference(a)
    assert torch.equal(expect, torch.zeros(n))
    assert torch.equal(out, expect)


def test_normalize_misaligned_and_in_place(dev):
    g = torch.Generator().manual_seed(5)
    a = torch.randn(10_001, generator=g)
    buf = torch.empty(10_002, device=dev)
    buf[1:] = a.to(dev)
    view = buf[1:]
    ppo_amd.normalize_advantages(view, out=view)
    torch.testing.assert_close(view.cpu(), ref.normalize_reference(a), rtol=1e-5, atol=1e-6)


def test_fused_gae_normalize_config2(dev):
    g = torch.Generator().manual_seed(24)
    T, N = 2048, 4096
    r = torch.randn(T, N, generator=g)
    v = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.01).to(torch.uint8)
    lv = torch.randn(N, generator=g)
    adv, ret, adv_n, stats = ppo_amd.gae_normalize(r.to(dev), v.to(dev), d.to(dev), lv.to(dev),
                                                   return_stats=True)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    n_ref = ref.normalize_reference(torch.from_numpy(a_ref).reshape(-1)).reshape(T, N)
    torch.testing.assert_close(adv_n.cpu(), n_ref, rtol=1e-5, atol=1e-6)
    x = a_ref.astype(np.float64)
    mean, std = stats.cpu().tolist()
    assert mean == pytest.approx(x.mean(), rel=1e-6, abs=1e-7)
    assert std == pytest.approx(x.std(ddof=1), rel=1e-6)
    # size-independent property: the normalised advantages have mean 0, std 1
    y = adv_n.double()
    assert abs(y.mean().item()) < 1e-6
    assert y.std().item() == pytest.approx(1.0, rel=1e-6)


def test_fused_matches_separate_ops(dev):
    g = torch.Generator().manual_seed(8)
    T, N = 333, 20
    r = torch.randn(T, N, generator=g).to(dev)
    v = torch.randn(T, N, generator=g).to(dev)
    d = (torch.rand(T, N, generator=g) < 0.05).to(torch.uint8).to(dev)
    adv, ret, adv_n = ppo_amd.gae_normalize(r, v, d)
    adv2, ret2 = ppo_amd.gae(r, v, d)
    assert torch.equal(adv, adv2) and torch.equal(ret, ret2)
    torch.testing.assert_close(adv_n, ppo_amd.normalize_advantages(adv2), rtol=1e-6, atol=1e-7)


# Advantages whose mean is large against their spread (|mean| / std up to
# 1e4): the normaliser's statistics must stay exact (the variance is not lost
# to the rounding of fp32 sums of squares).  Checked against fp64 statistics
# of the same advantages: the mean within one fp32 ulp (torch's own fp32
# reduction may land on the neighbouring float), the std within 1e-6
# relative, and adv_n = (adv - mean) / (std + eps) evaluated with the
# reported statistics.
OFFSET_ROUTES = [
    (2048, 4096, True),    # resident pass
    (2048, 4096, False),   # strip walk
    (16_384, 64, False),   # span passes
    (512, 259, False),     # unaligned N: tile passes
]


@pytest.mark.parametrize("mu", [1e2, 1e3, 1e4])
@pytest.mark.parametrize("T,N,resident", OFFSET_ROUTES)
def test_gae_normalize_large_mean(dev, monkeypatch, T, N, resident, mu):
    if not resident:
        monkeypatch.setenv("PPO_AMD_GAE_RESIDENT", "0")
    g = torch.Generator().manual_seed(int(mu) + N)
    r = mu + torch.randn(T, N, generator=g)
    v = torch.zeros(T, N)
    d = torch.ones(T, N, dtype=torch.uint8)  # every step done: adv = r - v
    print(f"gae_normalize large mean T={T} N={N} resident={resident} mu={mu}", flush=True)
    adv, _, adv_n, stats = ppo_amd.gae_normalize(r.to(dev), v.to(dev), d.to(dev), None, 0.99,
                                                 0.95, return_stats=True)
    a64 = adv.cpu().double()
    mean64, std64 = a64.mean().item(), a64.std().item()
    mean_f, std_f = stats.cpu().tolist()
    assert abs(mean_f - mean64) <= np.spacing(np.float32(abs(mean64))), (mean_f, mean64)
    assert std_f == pytest.approx(std64, rel=1e-6), (std_f, std64)
    a = adv.cpu()
    want = (a - torch.tensor(mean_f)) / (torch.tensor(std_f) + torch.tensor(1e-8))
    torch.testing.assert_close(adv_n.cpu(), want, rtol=1e-6, atol=1e-6)
