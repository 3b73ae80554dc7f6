"""GPU parity of the fused PPO loss kernels against the reference loss and
torch autograd on the CPU (oracle.loss_categorical_reference /
loss_gaussian_reference, which run ppo.py:150-169's own torch calls).

Tolerances (the benchmark's stated bar): loss scalars rel 1e-5; gradients rel 1e-4 per element
with an absolute floor of 1e-5 * max|g_ref| for elements near zero (the
gradient of a softmax row sums to zero, so some entries are cancellations).
"""

import math
import os

import numpy as np
import pytest
import torch

import ppo_amd
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ("loss", "policy", "value", "entropy", "approx_kl", "clipfrac")


def assert_grad_close(got, expect, rtol=1e-4, floor=1e-5):
    got = got.detach().cpu().double()
    expect = expect.detach().cpu().double()
    atol = floor * float(expect.abs().max()) if expect.numel() else 0.0
    torch.testing.assert_close(got, expect, rtol=rtol, atol=atol)


EDGE_ULPS = 8


def clip_edge_rows(ratio, lp, old_lp, clip=0.2, ulps=EDGE_ULPS):
    """Rows whose oracle ratio lies within `ulps` fp32 ulps of the log-probs
    (relative) of a clip bound 1 -/+ clip.  The clipped surrogate's gradient
    is discontinuous there: a log-prob summed in another order (torch's
    vectorised reduction against the kernel's dim loop) moves lp by an ulp or
    so, hence the ratio by that much relative, and can put the row on the
    other side of the bound, switching its policy gradient between the
    unclipped value, half of it (torch.minimum's tie) and zero.  Such rows
    are checked against those one-sided gradients (assert_edge_rows) instead
    of the oracle's own choice; every other row is held to the usual bar."""
    r = ratio.detach().cpu().double()
    m = torch.maximum(lp.detach().cpu().double().abs(), old_lp.detach().cpu().double().abs())
    band = ulps * m.clamp_min(1.0) * 2.0**-23
    return ((r - (1.0 - clip)).abs() <= band * r) | ((r - (1.0 + clip)).abs() <= band * r)


def assert_rows_close(got, expect, edge):
    keep = ~edge
    got = got.detach().cpu().double()
    expect = expect.detach().cpu().double()
    assert_grad_close(got[keep], expect[keep])
    print(f"  {int(edge.sum())} of {edge.numel()} rows within {EDGE_ULPS} ulps of a clip bound",
          flush=True)


def assert_edge_rows(got, candidates, edge, floor):
    """Each edge row equals one of its one-sided gradients: candidates is
    [k, n_edge, width] (k = clipped, tie, unclipped), compared at the usual
    per-element bar (rel 1e-4, absolute floor `floor`)."""
    if not bool(edge.any()):
        return
    g = got.detach().cpu().double()[edge]
    err = (g[None] - candidates).abs()
    lim = 1e-4 * candidates.abs() + floor
    ok = (err <= lim).all(dim=2).any(dim=0)
    assert bool(ok.all()), f"{int((~ok).sum())} edge rows match no one-sided gradient"


def cat_edge_candidates(logits, actions, adv, ratio, edge, ec=0.01):
    """d loss / d logits of the edge rows with the policy term's lp-gradient
    g in {0, -A r / 2, -A r} (clipped, tie, unclipped) and the entropy term,
    in fp64: [g (onehot - p) + ec p (log p + H)] / B."""
    B = logits.shape[0]
    z = logits.detach().cpu().double()[edge]
    logp = torch.log_softmax(z, -1)
    p = logp.exp()
    H = -(p * logp).sum(1, keepdim=True)
    onehot = torch.nn.functional.one_hot(actions.long().cpu()[edge], z.shape[1]).double()
    ent = ec * p * (logp + H)
    full = (-adv.cpu().double()[edge] * ratio.detach().cpu().double()[edge])[:, None]
    return torch.stack([(g * (onehot - p) + ent) / B for g in (0.0 * full, 0.5 * full, full)])


def gauss_edge_candidates(mu, log_std, acts, adv, ratio, edge):
    """d loss / d mu of the edge rows for g in {0, -A r / 2, -A r}:
    g (a - mu) / sigma^2 / B (the entropy does not depend on mu)."""
    B = mu.shape[0]
    var = (2.0 * log_std.detach().cpu().double()).exp()
    dlp = (acts.cpu().double()[edge] - mu.cpu().double()[edge]) / var
    full = (-adv.cpu().double()[edge] * ratio.detach().cpu().double()[edge])[:, None]
    return torch.stack([g * dlp / B for g in (0.0 * full, 0.5 * full, full)])


def assert_fixture_scalars(scalars, z):
    o = {k: torch.tensor(float(z["scalars"][i])) for i, k in enumerate(NAMES)}
    o["dvalues"] = torch.from_numpy(z["dvalues"])
    assert_scalars_close(scalars, o)


def assert_scalars_close(scalars, o, rtol=1e-5, edge_rows=0, lp_scale=1.0):
    """The reference's scalars (loss, policy, value, entropy) to rel 1e-5.
    approx_kl = mean(old_lp - lp) is a build-only diagnostic and a
    cancellation: each fp32 log-prob carries rounding of ~1e-7 of its
    magnitude (lp_scale: the largest |log-prob|, ~log A for categorical
    policies), so it is held to max(1, lp_scale) x 1e-6 absolute; clipfrac
    counts rows and may differ by a row whose ratio sits within an ulp of the
    clip bound."""
    s = scalars.detach().cpu()
    for i, k in enumerate(NAMES):
        e = o[k].item()
        if k == "approx_kl":
            assert s[i].item() == pytest.approx(e, abs=1e-6 * max(1.0, lp_scale)), k
        elif k == "clipfrac":
            slack = (2.0 + edge_rows) / o["dvalues"].numel()
            assert s[i].item() == pytest.approx(e, abs=slack + 1e-7), k
        else:
            assert s[i].item() == pytest.approx(e, rel=rtol, abs=1e-7), k


def cat_inputs(B, A, seed, act_dtype=torch.int32):
    """Configuration 4's distributions: logits ~ N(0,1); actions sampled from
    softmax(old_logits), old_logits = logits + N(0, 0.05); adv, ret, old
    values ~ N(0,1); values = old values + N(0, 0.1)."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, A, generator=g)
    old_logits = logits + 0.05 * torch.randn(B, A, generator=g)
    actions = torch.multinomial(torch.softmax(old_logits, -1), 1, generator=g).squeeze(1)
    old_lp = torch.log_softmax(old_logits, -1).gather(1, actions[:, None]).squeeze(1)
    adv = torch.randn(B, generator=g)
    ret = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    val = old_v + 0.1 * torch.randn(B, generator=g)
    return logits, actions.to(act_dtype), old_lp, adv, ret, val, old_v


def run_cat(dev, B, A, seed, vf_clip=0.2, act_dtype=torch.int32, inputs=None):
    inp = inputs if inputs is not None else cat_inputs(B, A, seed, act_dtype)
    logits, actions, old_lp, adv, ret, val, old_v = inp
    print(f"loss_cat B={B} A={A} vf_clip={vf_clip} act={actions.dtype}", flush=True)
    scalars, dlogits, dvalues = ppo_amd.ppo_loss_discrete_fused(
        logits.to(dev), actions.to(dev), old_lp.to(dev), adv.to(dev), ret.to(dev),
        val.to(dev), old_v.to(dev), 0.2, vf_clip, 0.5, 0.01,
    )
    o = ref.loss_categorical_reference(logits, actions, old_lp, adv, ret, val, old_v,
                                       0.2, vf_clip, 0.5, 0.01)
    lp = torch.log_softmax(logits, -1).gather(1, actions.long()[:, None]).squeeze(1)
    edge = clip_edge_rows(o["ratio"], lp, old_lp)
    assert_scalars_close(scalars, o, edge_rows=int(edge.sum()))
    assert_rows_close(dlogits, o["dlogits"], edge)
    assert_edge_rows(dlogits, cat_edge_candidates(logits, actions, adv, o["ratio"], edge), edge,
                     1e-5 * float(o["dlogits"].abs().max()))
    assert_grad_close(dvalues, o["dvalues"])
    return scalars, dlogits, dvalues


def test_golden_fixture_cat(dev):
    z = np.load(os.path.join(GOLDEN, "loss_cat_small.npz"))
    t = lambda k: torch.from_numpy(z[k]).to(dev)  # noqa: E731
    scalars, dlogits, dvalues = ppo_amd.ppo_loss_discrete_fused(
        t("logits"), t("actions"), t("old_log_probs"), t("advantages"), t("returns"),
        t("values"), t("old_values"), float(z["clip_ratio"]), float(z["vf_clip"]),
        float(z["value_coef"]), float(z["entropy_coef"]),
    )
    assert_fixture_scalars(scalars, z)
    assert_grad_close(dlogits, torch.from_numpy(z["dlogits"]))
    assert_grad_close(dvalues, torch.from_numpy(z["dvalues"]))


@pytest.mark.parametrize("B,A", [(1, 2), (7, 2), (256, 2), (257, 18), (1000, 18), (3, 1),
                                 (300, 5), (511, 33), (777, 48)])
@pytest.mark.parametrize("vf_clip", [None, 0.2])
def test_cat_row_kernel(dev, B, A, vf_clip):
    run_cat(dev, B, A, seed=B * 131 + A, vf_clip=vf_clip)


@pytest.mark.parametrize("A", [2, 3, 5, 6, 7, 9, 18, 1, 10, 13, 19, 4, 8, 12, 16, 20])
def test_cat_each_width_specialisation(dev, A):
    """Exact-width, predicated-width and LDS-pass forms of the row kernel,
    with a final partial tile (B not a multiple of 256)."""
    run_cat(dev, 2 * 256 * 9 + 77, A, seed=A, vf_clip=0.2)


@pytest.mark.parametrize("B,A", [(5, 49), (300, 64), (300, 100), (1025, 257)])
def test_cat_wave_kernel(dev, B, A):
    """A > 64 goes through the wave-per-row kernel."""
    run_cat(dev, B, A, seed=B + A, vf_clip=0.2)


def test_cat_int64_actions(dev):
    run_cat(dev, 1000, 18, seed=3, act_dtype=torch.int64)


def test_cat_ties_and_zero_advantage(dev):
    """ratio == 1 exactly (old_lp == lp) and adv == 0 rows hit the 1/2-1/2
    tie rule of torch.minimum; v - v_old at the clip bound hits clamp's
    inclusive edge."""
    B, A = 512, 6
    logits, actions, old_lp, adv, ret, val, old_v = cat_inputs(B, A, seed=4)
    lp = torch.log_softmax(logits, -1).gather(1, actions.long()[:, None]).squeeze(1)
    old_lp[: B // 2] = lp[: B // 2]
    adv[::7] = 0.0
    run_cat(dev, B, A, seed=0, inputs=(logits, actions, old_lp, adv, ret, val, old_v))


def _exact_bound_old_lp(lp, c, want=8):
    """fp32 old log-probs for which torch's fp32 ratio exp(lp - old_lp) is
    exactly fp32(c), with exp of that fp32 difference within 0.25 ulp of c in
    fp64 (so an exp with error below a quarter ulp lands on c too)."""
    c32 = torch.tensor(c, dtype=torch.float32)
    lp32 = torch.tensor(lp, dtype=torch.float32)
    ulp_c = float(torch.nextafter(c32, torch.tensor(2.0)) - c32)
    x0 = (lp32.double() - math.log(float(c32))).float()
    found = []
    for direction in (-100.0, 100.0):
        x = x0
        for _ in range(256):
            d = lp32 - x
            if torch.exp(d) == c32 and abs(math.exp(float(d)) - float(c32)) < 0.25 * ulp_c:
                found.append(float(x))
            x = torch.nextafter(x, torch.tensor(direction))
    found = sorted(set(found))[:want]
    assert found, f"no exact-bound old log-prob for {c}"
    return found


def test_cat_ratio_exactly_on_the_clip_bounds(dev):
    """The fp32 ratio lands exactly on 1 - clip and 1 + clip (uniform logits,
    so lp = -log 2 in the kernel and in torch alike; old_lp chosen so that
    exp(lp - old_lp) rounds to the bound).  torch.clamp passes the gradient at
    its inclusive bounds and torch.minimum splits a tie 1/2-1/2, so the
    reference's policy gradient there is the full unclipped one: the kernel
    must give exactly that, not zero (which exclusive bounds would give)."""
    A = 2
    lp = float(torch.log_softmax(torch.zeros(A), -1)[0])
    rows = []
    for c in (0.8, 1.2):
        for olp in _exact_bound_old_lp(lp, c):
            for a in (1.5, -0.75):
                rows.append((olp, a))
    B = len(rows)
    logits = torch.zeros(B, A)
    actions = torch.tensor([i % A for i in range(B)], dtype=torch.int32)
    old_lp = torch.tensor([r[0] for r in rows], dtype=torch.float32)
    adv = torch.tensor([r[1] for r in rows], dtype=torch.float32)
    g = torch.Generator().manual_seed(13)
    ret = torch.randn(B, generator=g)
    val = torch.randn(B, generator=g)
    print(f"loss_cat exact clip bounds B={B}", flush=True)
    scalars, dlogits, dvalues = ppo_amd.ppo_loss_discrete_fused(
        logits.to(dev), actions.to(dev), old_lp.to(dev), adv.to(dev), ret.to(dev), val.to(dev),
        None, 0.2, None, 0.5, 0.01)
    o = ref.loss_categorical_reference(logits, actions, old_lp, adv, ret, val, None,
                                       0.2, None, 0.5, 0.01)
    r = o["ratio"]
    assert bool(((r == torch.tensor(0.8)) | (r == torch.tensor(1.2))).all())
    # the reference's rows carry the full policy gradient -A r (onehot - p) / B
    full = cat_edge_candidates(logits, actions, adv, r, torch.ones(B, dtype=torch.bool))[2]
    torch.testing.assert_close(o["dlogits"].double(), full, rtol=1e-6, atol=1e-9)
    assert_grad_close(dlogits, o["dlogits"])
    assert_scalars_close(scalars, o)


@pytest.mark.parametrize("A", [2, 5, 18, 33, 100])
def test_cat_masked_logits(dev, A):
    """Action masking by -inf logits (never at the taken action), as
    torch.distributions.Categorical accepts it: finite loss, entropy and
    gradients, zero gradient at the masked logits.  A = 2, 5, 18 take the
    exact-width wave tiles, 33 the LDS-pass form and 100 the wave-per-row
    kernel."""
    B = 1000
    g = torch.Generator().manual_seed(700 + A)
    logits = torch.randn(B, A, generator=g)
    mask = torch.rand(B, A, generator=g) < 0.3
    old_logits = (logits + 0.05 * torch.randn(B, A, generator=g)).masked_fill(mask, -float("inf"))
    keep = (~mask).any(1)
    old_logits[~keep, 0] = 0.0  # (every row keeps at least one action)
    mask[~keep, 0] = False
    actions = torch.multinomial(torch.softmax(old_logits, -1), 1, generator=g).squeeze(1)
    old_lp = torch.log_softmax(old_logits, -1).gather(1, actions[:, None]).squeeze(1)
    logits = logits.masked_fill(mask, -float("inf"))
    assert not mask.gather(1, actions[:, None]).any()
    adv = torch.randn(B, generator=g)
    ret = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    val = old_v + 0.1 * torch.randn(B, generator=g)
    inputs = (logits, actions.to(torch.int32), old_lp, adv, ret, val, old_v)
    scalars, dlogits, _ = run_cat(dev, B, A, seed=0, inputs=inputs)
    assert torch.isfinite(scalars).all()
    dl = dlogits.cpu()
    assert torch.isfinite(dl).all()
    assert (dl[mask] == 0).all()


@pytest.mark.parametrize("scale", [30.0, 100.0])
@pytest.mark.parametrize("A", [2, 18, 33])
def test_cat_peaked_logits(dev, A, scale):
    """Logits of large magnitude (near-deterministic policies, probabilities
    underflowing to 0 in fp32): the kernel's max-shifted exponentials and
    closed-form gradient against torch's log_softmax-based Categorical.  (At
    |logits| ~ 1e3 the fp32 rounding of z - max itself, an ulp of ~6e-5, moves
    small probabilities by ~1e-4 relative in either implementation, beyond
    the 1e-4 gradient tolerance.)"""
    logits, actions, old_lp, adv, ret, val, old_v = cat_inputs(1000, A, seed=int(scale) + A)
    logits = logits * scale
    old_lp = torch.log_softmax(logits, -1).gather(1, actions.long()[:, None]).squeeze(1) + \
        0.05 * torch.randn(1000, generator=torch.Generator().manual_seed(A))
    run_cat(dev, 1000, A, seed=0, inputs=(logits, actions, old_lp, adv, ret, val, old_v))


def test_cat_misaligned_logits(dev):
    B, A = 300, 18
    inp = cat_inputs(B, A, seed=6)
    logits = inp[0]
    buf = torch.empty(B * A + 1, device=dev)
    buf[1:] = logits.reshape(-1).to(dev)
    lg = buf[1:].view(B, A)
    _, actions, old_lp, adv, ret, val, old_v = inp
    scalars, dlogits, dvalues = ppo_amd.ppo_loss_discrete_fused(
        lg, actions.to(dev), old_lp.to(dev), adv.to(dev), ret.to(dev), val.to(dev), None,
    )
    o = ref.loss_categorical_reference(logits, actions, old_lp, adv, ret, val)
    assert_scalars_close(scalars, o)
    assert_grad_close(dlogits, o["dlogits"])


def test_cat_config4_full_size(dev):
    """Configuration 4: B=1,048,576, A=18, vf_clip=0.2."""
    scalars, dlogits, _ = run_cat(dev, 1_048_576, 18, seed=24, vf_clip=0.2)
    # size-independent invariant: each softmax row of the gradient sums to 0
    rows = dlogits.double().sum(1).abs().max().item()
    assert rows < 1e-9


def test_cat_autograd_matches_fused(dev):
    B, A = 999, 4
    logits, actions, old_lp, adv, ret, val, old_v = cat_inputs(B, A, seed=8)
    lg = logits.to(dev).requires_grad_(True)
    vv = val.to(dev).requires_grad_(True)
    loss, stats = ppo_amd.ppo_loss_discrete(lg, actions.to(dev), old_lp.to(dev), adv.to(dev),
                                            ret.to(dev), vv)
    (2.0 * loss).backward()
    o = ref.loss_categorical_reference(logits, actions, old_lp, adv, ret, val)
    assert loss.item() == pytest.approx(o["loss"].item(), rel=1e-5)
    assert_grad_close(lg.grad, 2.0 * o["dlogits"])
    assert_grad_close(vv.grad, 2.0 * o["dvalues"])
    assert stats["entropy"].item() == pytest.approx(o["entropy"].item(), rel=1e-5)


def test_cat_out_of_range_action(dev):
    B, A = 16, 3
    logits, actions, old_lp, adv, ret, val, _ = cat_inputs(B, A, seed=9)
    actions[5] = 3
    args = [x.to(dev) for x in (logits, actions, old_lp, adv, ret, val)]
    with pytest.raises(ValueError):
        ppo_amd.ppo_loss_discrete_fused(*args, validate_args=True)
    scalars, _, _ = ppo_amd.ppo_loss_discrete_fused(*args)
    assert torch.isnan(scalars[0]).item()


# ---------------------------------------------------------------------------
# Gaussian
# ---------------------------------------------------------------------------
def gauss_inputs(B, D, seed):
    """Configuration 5's distributions: mu ~ N(0,1); log_std ~ U(-1,0);
    actions ~ N(mu_old, exp(log_std)), mu_old = mu + N(0, 0.05)."""
    g = torch.Generator().manual_seed(seed)
    mu = torch.randn(B, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0
    mu_old = mu + 0.05 * torch.randn(B, D, generator=g)
    acts = mu_old + log_std.exp() * torch.randn(B, D, generator=g)
    old_lp = torch.distributions.Normal(mu_old, log_std.exp()).log_prob(acts).sum(-1)
    adv = torch.randn(B, generator=g)
    ret = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    val = old_v + 0.1 * torch.randn(B, generator=g)
    return mu, log_std, acts, old_lp, adv, ret, val, old_v


def run_gauss(dev, B, D, seed, vf_clip=0.2, inputs=None):
    inp = inputs if inputs is not None else gauss_inputs(B, D, seed)
    print(f"loss_gauss B={B} D={D} vf_clip={vf_clip}", flush=True)
    mu, log_std, acts, old_lp, adv, ret, val, old_v = inp
    scalars, dmu, dls, dv = ppo_amd.ppo_loss_gaussian_fused(
        *[x.to(dev) for x in inp], 0.2, vf_clip, 0.5, 0.01
    )
    o = ref.loss_gaussian_reference(*inp, 0.2, vf_clip, 0.5, 0.01)
    lp = torch.distributions.Normal(mu, log_std.exp()).log_prob(acts).sum(-1)
    edge = clip_edge_rows(o["ratio"], lp, old_lp)
    assert_scalars_close(scalars, o, edge_rows=int(edge.sum()),
                         lp_scale=float(old_lp.abs().max()) / 3.0)
    assert_rows_close(dmu, o["dmu"], edge)
    assert_edge_rows(dmu, gauss_edge_candidates(mu, log_std, acts, adv, o["ratio"], edge), edge,
                     1e-5 * float(o["dmu"].abs().max()))
    # dlog_std sums over rows: an edge row may add or drop its policy term
    # |A| r ((x - mu)^2 / sigma^2 - 1) / B (x1.5 at a tie), so the
    # tolerance widens by exactly that much for those rows
    r = o["ratio"].double()
    z2 = ((acts.double() - mu.double()) / log_std.double().exp()) ** 2
    extra = ((adv.double().abs() * r * 1.5)[:, None] * (z2 - 1).abs())[edge].sum(0) / B
    diff = (dls.detach().cpu().double() - o["dlog_std"].double()).abs()
    lim = 1e-4 * o["dlog_std"].double().abs() + 1e-5 * float(o["dlog_std"].abs().max()) + extra
    assert bool((diff <= lim).all()), (diff, lim)
    assert_grad_close(dv, o["dvalues"])


def test_golden_fixture_gauss(dev):
    z = np.load(os.path.join(GOLDEN, "loss_gauss_small.npz"))
    t = lambda k: torch.from_numpy(z[k]).to(dev)  # noqa: E731
    scalars, dmu, dls, dv = ppo_amd.ppo_loss_gaussian_fused(
        t("mu"), t("log_std"), t("actions"), t("old_log_probs"), t("advantages"),
        t("returns"), t("values"), t("old_values"), float(z["clip_ratio"]),
        float(z["vf_clip"]), float(z["value_coef"]), float(z["entropy_coef"]),
    )
    assert_fixture_scalars(scalars, z)
    assert_grad_close(dmu, torch.from_numpy(z["dmu"]))
    assert_grad_close(dls, torch.from_numpy(z["dlog_std"]))
    assert_grad_close(dv, torch.from_numpy(z["dvalues"]))


@pytest.mark.parametrize("B,D", [(1, 1), (5, 6), (256, 6), (1000, 6), (333, 17), (300, 24)])
@pytest.mark.parametrize("vf_clip", [None, 0.2])
def test_gauss(dev, B, D, vf_clip):
    run_gauss(dev, B, D, seed=B * 7 + D, vf_clip=vf_clip)


@pytest.mark.parametrize("shift", [-6.0, 3.0])
@pytest.mark.parametrize("D", [1, 6, 17])
def test_gauss_extreme_log_std(dev, D, shift):
    """Very narrow (sigma ~ 1e-3) and very wide (sigma ~ 20) policies: the
    same checks as test_gauss with log_std shifted by `shift` and the actions
    drawn at that scale."""
    B = 1000
    g = torch.Generator().manual_seed(int(shift * 10) + D)
    mu = torch.randn(B, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0 + shift
    mu_old = mu + 0.05 * log_std.exp() * torch.randn(B, D, generator=g)
    acts = mu_old + log_std.exp() * torch.randn(B, D, generator=g)
    old_lp = torch.distributions.Normal(mu_old, log_std.exp()).log_prob(acts).sum(-1)
    adv, ret, old_v = (torch.randn(B, generator=g) for _ in range(3))
    val = old_v + 0.1 * torch.randn(B, generator=g)
    run_gauss(dev, B, D, seed=0, inputs=(mu, log_std, acts, old_lp, adv, ret, val, old_v))


@pytest.mark.parametrize("D", [1, 2, 3, 4, 5, 6, 7, 8, 9, 13, 16, 17, 24])
def test_gauss_each_width_specialisation(dev, D):
    """Exact-width and predicated-width register kernels, final partial tile."""
    run_gauss(dev, 2 * 256 * 9 + 77, D, seed=100 + D)


def test_gauss_misaligned_mu(dev):
    B, D = 700, 6
    inp = gauss_inputs(B, D, seed=12)
    mu = inp[0]
    buf = torch.empty(B * D + 1, device=dev)
    buf[1:] = mu.reshape(-1).to(dev)
    args = [buf[1:].view(B, D)] + [x.to(dev) for x in inp[1:]]
    scalars, dmu, dls, dv = ppo_amd.ppo_loss_gaussian_fused(*args, 0.2, 0.2, 0.5, 0.01)
    o = ref.loss_gaussian_reference(*inp, 0.2, 0.2, 0.5, 0.01)
    assert_scalars_close(scalars, o)
    assert_grad_close(dmu, o["dmu"])
    assert_grad_close(dls, o["dlog_std"])


def test_gauss_config5_full_size(dev):
    """Configuration 5: B=2,097,152, D=6, vf_clip=0.2."""
    run_gauss(dev, 2_097_152, 6, seed=24)


def test_gauss_autograd(dev):
    mu, log_std, acts, old_lp, adv, ret, val, old_v = gauss_inputs(500, 6, seed=11)
    m = mu.to(dev).requires_grad_(True)
    ls = log_std.to(dev).requires_grad_(True)
    vv = val.to(dev).requires_grad_(True)
    loss, _ = ppo_amd.ppo_loss_gaussian(m, ls, acts.to(dev), old_lp.to(dev), adv.to(dev),
                                        ret.to(dev), vv)
    loss.backward()
    o = ref.loss_gaussian_reference(mu, log_std, acts, old_lp, adv, ret, val)
    assert_grad_close(m.grad, o["dmu"])
    assert_grad_close(ls.grad, o["dlog_std"])
    assert_grad_close(vv.grad, o["dvalues"])


# ---------------------------------------------------------------------------
# Seeded sweep over row counts on both sides of the persistent grid's capacity
# (262,144 rows per round at 4096 waves x 64 rows), ragged final tiles, and
# the width specialisations, action dtypes and value-clip settings.
# ---------------------------------------------------------------------------
def _loss_sweep(count, widths, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        # half the cases past one grid round (200k-700k rows), half 1..~16k rows
        B = int(rng.uniform(2e5, 7e5)) if rng.random() < 0.5 else int(2 ** rng.uniform(0, 14))
        cases.append((B, int(rng.choice(widths)), bool(rng.random() < 0.5),
                      bool(rng.random() < 0.3)))
    return cases


@pytest.mark.parametrize("B,A,clip,i64", _loss_sweep(12, [1, 2, 6, 18, 33, 100], 7))
def test_cat_row_count_sweep(dev, B, A, clip, i64):
    run_cat(dev, B, A, seed=B + 1000 * A, vf_clip=0.2 if clip else None,
            act_dtype=torch.int64 if i64 else torch.int32)


@pytest.mark.parametrize("B,D,clip,_", _loss_sweep(8, [1, 6, 8, 9, 17], 11))
def test_gauss_row_count_sweep(dev, B, D, clip, _):
    run_gauss(dev, B, D, seed=B + 1000 * D, vf_clip=0.2 if clip else None)


# ---------------------------------------------------------------------------
# Past 2^31 elements: B = 120,000,000 rows x A = 18 (2.16e9 logits, ~21 GB on
# the device), checked against the same entry point on chunks below 2^31
# elements (each of which the tests above tie to the oracle).  Rows are
# independent except for the 1/B in every gradient and the means, so a row's
# gradient times B must match between the whole call and its chunk's call,
# and each scalar must equal the B-weighted mean of the chunks' scalars.
# ---------------------------------------------------------------------------
def test_cat_past_2_31_elements(dev):
    B, A, chunks = 120_000_000, 18, 4
    print(f"loss_cat B={B} A={A} (past 2^31 elements)", flush=True)
    g = torch.Generator(device=dev).manual_seed(31)
    logits = torch.randn(B, A, device=dev, generator=g)
    actions = torch.randint(0, A, (B,), device=dev, generator=g, dtype=torch.int32)
    old_lp = torch.log_softmax(logits, -1).gather(1, actions[:, None].long()).squeeze(1)
    old_lp += 0.05 * torch.randn(B, device=dev, generator=g)
    adv, ret, old_v = (torch.randn(B, device=dev, generator=g) for _ in range(3))
    val = old_v + 0.1 * torch.randn(B, device=dev, generator=g)
    scalars, dlogits, dv = ppo_amd.ppo_loss_discrete_fused(logits, actions, old_lp, adv, ret, val,
                                                           old_v, 0.2, 0.2, 0.5, 0.01)
    torch.cuda.synchronize(dev)
    assert torch.isfinite(scalars).all()
    weighted = torch.zeros(6, dtype=torch.float64)
    step = B // chunks
    for c in range(chunks):
        sl = slice(c * step, B if c == chunks - 1 else (c + 1) * step)
        bc = sl.stop - sl.start
        sc, dlc, dvc = ppo_amd.ppo_loss_discrete_fused(
            logits[sl], actions[sl], old_lp[sl], adv[sl], ret[sl], val[sl], old_v[sl],
            0.2, 0.2, 0.5, 0.01)
        weighted += sc.double().cpu() * bc / B
        # gradients x rows: identical up to fp32 rounding of the 1/B factors
        for big, small in ((dlogits[sl], dlc), (dv[sl], dvc)):
            x = big.double() * B
            y = small.double() * bc
            tol = 1e-5 * y.abs() + 1e-6 * float(y.abs().max())
            assert bool(((x - y).abs() <= tol).all()), c
        del sc, dlc, dvc
    # every scalar is linear in the chunks' (fp32-rounded) means
    torch.testing.assert_close(scalars.double().cpu(), weighted, rtol=2e-5, atol=1e-6)


def test_empty_batches_raise_like_the_reference(dev):
    """A minibatch of no rows: the reference's Categorical / Normal on an
    empty batch raises (torch cannot validate a [0, A] tensor, and the means
    of ppo.py:159-167 would be NaN); the fused losses raise ValueError before
    any launch, also for A = 0 or D = 0."""
    e = torch.zeros(0, device=dev)
    with pytest.raises(ValueError, match="B > 0"):
        ppo_amd.ppo_loss_discrete(torch.zeros(0, 18, device=dev),
                                  torch.zeros(0, dtype=torch.int32, device=dev), e, e, e, e)
    with pytest.raises(ValueError, match="A > 0"):
        z = torch.zeros(4, device=dev)
        ppo_amd.ppo_loss_discrete(torch.zeros(4, 0, device=dev),
                                  torch.zeros(4, dtype=torch.int32, device=dev), z, z, z, z)
    with pytest.raises(ValueError, match="B > 0"):
        ppo_amd.ppo_loss_gaussian(torch.zeros(0, 6, device=dev), torch.zeros(6, device=dev),
                                  torch.zeros(0, 6, device=dev), e, e, e, e)
    with pytest.raises(Exception):
        torch.distributions.Categorical(logits=torch.zeros(0, 18)).log_prob(
            torch.zeros(0, dtype=torch.int64))
