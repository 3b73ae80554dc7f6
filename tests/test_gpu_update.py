"""GPU parity of the update-loop kernels: the fused minibatch gather
(ppo.py:132-139) and clip_grad_norm_ + Adam (ppo.py:170-171) against torch
on the same data.

Tolerances: the gather is a byte copy (exact).  ClippedAdam follows torch's
multi-tensor Adam operation by operation in fp32; the global norm is reduced
in a different order, so parameters are compared at rel 2e-6 / abs 1e-7 after
several steps and the returned norm at rel 1e-6.
"""

import pytest
import torch

import ppo_amd

pytestmark = pytest.mark.gpu


def test_gather_rows_matches_indexing(dev):
    g = torch.Generator().manual_seed(0)
    n, B = 10_000, 3_333
    obs = torch.randn(n, 4, generator=g).to(dev)
    acts32 = torch.randint(0, 18, (n,), generator=g, dtype=torch.int32).to(dev)
    acts64 = torch.randint(0, 18, (n,), generator=g).to(dev)
    lp = torch.randn(n, generator=g).to(dev)
    mu = torch.randn(n, 6, generator=g).to(dev)
    idx = torch.randperm(n, generator=g)[:B].to(dev)
    outs = ppo_amd.gather_rows(idx, obs, acts32, acts64, lp, mu)
    for o, a in zip(outs, (obs, acts32, acts64, lp, mu)):
        assert o.dtype == a.dtype and o.shape == (B,) + a.shape[1:]
        assert torch.equal(o, a[idx])


def test_gather_rows_out_of_range_gives_zero_rows(dev):
    a = torch.arange(40, dtype=torch.float32, device=dev).reshape(10, 4)
    idx = torch.tensor([0, 9, 10, -1, 3], device=dev)
    (o,) = ppo_amd.gather_rows(idx, a)
    assert torch.equal(o[[0, 1, 4]], a[[0, 9, 3]])
    assert torch.equal(o[[2, 3]], torch.zeros(2, 4, device=dev))


def _make_params(dev, seed, shapes):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g).to(dev).requires_grad_(True) for s in shapes]


@pytest.mark.parametrize("capturable", [False, True])
@pytest.mark.parametrize("max_norm", [0.5, 1e6, 0.0])
def test_clipped_adam_matches_torch(dev, max_norm, capturable):
    shapes = [(64, 4), (64,), (64, 64), (64,), (2, 64), (2,), (10_000,), (3, 5, 7)]
    p_ref = _make_params(dev, 1, shapes)
    p_got = [p.detach().clone().requires_grad_(True) for p in p_ref]
    opt_ref = torch.optim.Adam(p_ref, lr=3e-4)
    opt_got = ppo_amd.ClippedAdam(p_got, lr=3e-4, max_grad_norm=max_norm,
                                 capturable=capturable)
    g = torch.Generator().manual_seed(2)
    for step in range(5):
        grads = [torch.randn(*s, generator=g).to(dev) * (0.1 + step) for s in shapes]
        for p, gr in zip(p_ref, grads):
            p.grad = gr.clone()
        for p, gr in zip(p_got, grads):
            p.grad = gr.clone()
        if max_norm > 0:
            norm_ref = torch.nn.utils.clip_grad_norm_(p_ref, max_norm)
        else:
            norm_ref = torch.linalg.vector_norm(
                torch.stack([torch.linalg.vector_norm(p.grad) for p in p_ref]))
        opt_ref.step()
        norm_got = opt_got.step()
        assert norm_got.item() == pytest.approx(norm_ref.item(), rel=1e-6)
        for a, b in zip(p_got, p_ref):
            torch.testing.assert_close(a, b, rtol=2e-6, atol=1e-7)
            torch.testing.assert_close(a.grad, b.grad, rtol=2e-6, atol=1e-9)
    for k, p in enumerate(p_ref):
        st = opt_ref.state[p]
        torch.testing.assert_close(opt_got.exp_avg[k], st["exp_avg"], rtol=2e-6, atol=1e-9)
        torch.testing.assert_close(opt_got.exp_avg_sq[k], st["exp_avg_sq"], rtol=2e-6,
                                   atol=1e-12)


def test_clipped_adam_skips_missing_grads(dev):
    p = _make_params(dev, 3, [(8,), (9,)])
    opt = ppo_amd.ClippedAdam(p, lr=1e-2, max_grad_norm=0.0)
    before = p[1].detach().clone()
    p[0].grad = torch.ones(8, device=dev)
    opt.step()
    assert torch.equal(p[1].detach(), before)
    assert opt.steps == [1, 0]


def test_copy_from_pinned(dev):
    """ppo_copy_from_pinned: pinned host -> device by a kernel launch; memory
    that is not pinned is refused before any launch."""
    import ctypes

    import numpy as np

    from ppo_amd import _lib, ops

    src = torch.randperm(10_000, generator=torch.Generator().manual_seed(3)).reshape(4, 2500)
    pinned = src.pin_memory()
    dst = torch.empty(4, 2500, dtype=torch.int64, device=dev)
    ops.copy_pinned_to_device(dst, pinned)
    assert torch.equal(dst.cpu(), src)
    with pytest.raises(ValueError):
        ops.copy_pinned_to_device(dst, src)  # not pinned: refused on the host side
    plain = np.arange(16, dtype=np.int32)
    rc = _lib.load().ppo_copy_from_pinned(dst.data_ptr(), plain.ctypes.data_as(ctypes.c_void_p),
                                          64, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.PPO_OK + 1  # PPO_ERR_INVALID_ARG: not pinned, nothing launched
    assert torch.equal(dst.cpu(), src)


@pytest.mark.parametrize("capturable", [False, True])
def test_clipped_adam_state_dict_round_trip_with_torch_adam(dev, capturable):
    """ClippedAdam.state_dict() has torch.optim.Adam's layout: a torch Adam
    loads it and continues with the same steps (and the reverse), and
    load_state_dict copies into the existing moment buffers."""
    torch.manual_seed(0)
    shapes = [(8, 4), (8,), (3, 8), (3,)]
    p1 = [torch.randn(s, device=dev, requires_grad=True) for s in shapes]
    p2 = [p.detach().clone().requires_grad_(True) for p in p1]
    opt = ppo_amd.ClippedAdam(p1, lr=1e-2, max_grad_norm=0.0, capturable=capturable)
    ref_opt = torch.optim.Adam(p2, lr=1e-2)
    for _ in range(3):
        grads = [torch.randn(s, device=dev) for s in shapes]
        for p, g in zip(p1, grads):
            p.grad = g.clone()
        for p, g in zip(p2, grads):
            p.grad = g.clone()
        opt.step()
        ref_opt.step()
    sd = opt.state_dict()
    assert sd["param_groups"][0]["params"] == [0, 1, 2, 3]
    fresh = torch.optim.Adam([p.detach().clone().requires_grad_(True) for p in p1], lr=1e-2)
    fresh.load_state_dict(sd)
    for i in range(4):
        torch.testing.assert_close(fresh.state[fresh.param_groups[0]["params"][i]]["exp_avg"],
                                   ref_opt.state[p2[i]]["exp_avg"], rtol=1e-5, atol=1e-7)
    buf = opt.exp_avg[0]
    opt2 = ppo_amd.ClippedAdam(p1, lr=1e-3, max_grad_norm=0.0, capturable=capturable)
    keep = opt2.exp_avg[0]
    opt2.load_state_dict(ref_opt.state_dict())
    assert opt2.exp_avg[0] is keep and opt2.lr == 1e-2
    assert opt2.step_count() == 3
    torch.testing.assert_close(opt2.exp_avg[0], buf, rtol=1e-5, atol=1e-7)


def test_keep_grads_zeroes_in_place(dev):
    p = torch.randn(4, device=dev, requires_grad=True)
    opt = ppo_amd.ClippedAdam([p])
    p.grad = torch.ones(4, device=dev)
    g = p.grad
    opt.keep_grads = True
    opt.zero_grad()
    assert p.grad is g and bool((g == 0).all())
    opt.keep_grads = False
    opt.zero_grad()
    assert p.grad is None
