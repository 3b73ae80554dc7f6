"""The allocation-free loss entry point (ppo_loss_cat_f32_noalloc) against
ppo_loss_cat_f32 with a caller workspace, both called through the C ABI on
the same inputs: scalars, dlogits and dvalues must be bit-identical.  Two
calls in a row, the second with a smaller input (the library's scratch keeps
the first call's partial sums, which must not leak into the second), then a
row width that takes the wave-per-row kernel and its larger grid."""

import ctypes

import pytest
import torch

from ppo_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(dev, B, A, seed, int64):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, A, generator=g)
    old = logits + 0.05 * torch.randn(B, A, generator=g)
    actions = torch.multinomial(torch.softmax(old, -1), 1, generator=g).squeeze(1)
    old_lp = torch.log_softmax(old, -1).gather(1, actions[:, None]).squeeze(1)
    adv = torch.randn(B, generator=g)
    ret = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    v = old_v + 0.1 * torch.randn(B, generator=g)
    actions = actions.to(torch.int64 if int64 else torch.int32)
    return [t.contiguous().to(dev) for t in (logits, actions, old_lp, adv, ret, v, old_v)]


def _run(lib, dev, B, A, seed, int64, vf_clip):
    logits, actions, old_lp, adv, ret, v, old_v = _inputs(dev, B, A, seed, int64)
    params = _lib.LossParams(0.2, vf_clip, 0.5, 0.01)
    stream = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for noalloc in (False, True):
        dlogits = torch.full_like(logits, float("nan"))
        dvalues = torch.full_like(v, float("nan"))
        scalars = torch.full((_lib.PPO_NUM_SCALARS,), float("nan"), device=dev)
        common = (logits.data_ptr(), B, A, actions.data_ptr(), int(int64), old_lp.data_ptr(),
                  adv.data_ptr(), ret.data_ptr(), v.data_ptr(), old_v.data_ptr(),
                  ctypes.byref(params), dlogits.data_ptr(), dvalues.data_ptr(),
                  scalars.data_ptr())
        if noalloc:
            code = lib.ppo_loss_cat_f32_noalloc(*common, stream)
        else:
            nbytes = lib.ppo_loss_cat_workspace_bytes(B, A)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            code = lib.ppo_loss_cat_f32(*common, ws.data_ptr(), nbytes, stream)
        _lib.check("ppo_loss_cat_f32_noalloc" if noalloc else "ppo_loss_cat_f32", code)
        torch.cuda.synchronize(dev)
        outs.append((scalars.cpu(), dlogits.cpu(), dvalues.cpu()))
    (s0, g0, v0), (s1, g1, v1) = outs
    assert torch.isfinite(s0).all()
    assert torch.equal(s0, s1), (s0, s1)
    assert torch.equal(g0, g1)
    assert torch.equal(v0, v1)


def test_noalloc_matches_workspace_entry_point(dev):
    lib = _lib.load()
    for B, A, seed, int64, vf_clip in (
        (1 << 20, 18, 1, False, 0.2),   # configuration 4's shape, persistent grid
        (10_007, 18, 2, True, 0.0),     # smaller: fewer workgroups than the first call
        (3_001, 64, 3, False, 0.2),     # wave-per-row kernel
        (257, 2, 4, False, 0.0),        # smaller again
    ):
        print(f"noalloc B={B} A={A} seed={seed} int64={int64} vf_clip={vf_clip}", flush=True)
        _run(lib, dev, B, A, seed, int64, vf_clip)


def test_noalloc_rejects_bad_arguments(dev):
    lib = _lib.load()
    params = _lib.LossParams(0.2, 0.0, 0.5, 0.01)
    assert lib.ppo_loss_cat_f32_noalloc(None, 0, 4, None, 0, None, None, None, None, None,
                                        ctypes.byref(params), None, None, None, None) == 1
