"""torch.ops.ppo_amd.* registration (ppo_amd/torch_ops.py), without a GPU:
schemas, fake (meta) implementations for torch.compile's tracing, and that a
CPU tensor is refused (no CPU fallback)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import ppo_amd  # noqa: F401  (registers the operators)

OPS = {
    "gae": "ppo_amd::gae(Tensor rewards, Tensor values, Tensor dones, Tensor? last_value, "
           "float gamma, float lam) -> (Tensor, Tensor)",
    "gae_normalize": "ppo_amd::gae_normalize(Tensor rewards, Tensor values, Tensor dones, "
                     "Tensor? last_value, float gamma, float lam, float eps) "
                     "-> (Tensor, Tensor, Tensor, Tensor)",
    "normalize_advantages": "ppo_amd::normalize_advantages(Tensor advantages, float eps) -> Tensor",
    "ppo_loss_discrete": "ppo_amd::ppo_loss_discrete(Tensor logits, Tensor actions, "
                         "Tensor old_log_probs, Tensor advantages, Tensor returns, Tensor values, "
                         "Tensor? old_values, float clip_ratio, float? vf_clip, float value_coef, "
                         "float entropy_coef) -> (Tensor, Tensor, Tensor)",
    "ppo_loss_gaussian": "ppo_amd::ppo_loss_gaussian(Tensor mu, Tensor log_std, Tensor actions, "
                         "Tensor old_log_probs, Tensor advantages, Tensor returns, Tensor values, "
                         "Tensor? old_values, float clip_ratio, float? vf_clip, float value_coef, "
                         "float entropy_coef) -> (Tensor, Tensor, Tensor, Tensor)",
}


@pytest.mark.parametrize("name", sorted(OPS))
def test_schema(name):
    assert str(getattr(torch.ops.ppo_amd, name).default._schema) == OPS[name]


def test_fake_shapes():
    with FakeTensorMode():
        T, N, B, A, D = 16, 8, 32, 5, 3
        dev = "cuda"
        r = torch.empty(T, N, device=dev)
        d = torch.empty(T, N, dtype=torch.uint8, device=dev)
        adv, ret = torch.ops.ppo_amd.gae(r, r, d, None, 0.99, 0.95)
        assert adv.shape == ret.shape == (T, N)
        adv, ret, adv_n, stats = torch.ops.ppo_amd.gae_normalize(r, r, d, None, 0.99, 0.95, 1e-8)
        assert adv_n.shape == (T, N) and stats.shape == (2,)
        assert torch.ops.ppo_amd.normalize_advantages(r, 1e-8).shape == (T, N)
        logits = torch.empty(B, A, device=dev)
        rows = torch.empty(B, device=dev)
        act = torch.empty(B, dtype=torch.int64, device=dev)
        sc, dl, dv = torch.ops.ppo_amd.ppo_loss_discrete(logits, act, rows, rows, rows, rows, None,
                                                         0.2, None, 0.5, 0.01)
        assert sc.shape == (6,) and dl.shape == (B, A) and dv.shape == (B,)
        mu = torch.empty(B, D, device=dev)
        ls = torch.empty(D, device=dev)
        sc, dmu, dls, dv = torch.ops.ppo_amd.ppo_loss_gaussian(mu, ls, mu, rows, rows, rows, rows,
                                                               None, 0.2, 0.2, 0.5, 0.01)
        assert dmu.shape == (B, D) and dls.shape == (D,) and dv.shape == (B,)


def test_cpu_tensors_are_refused():
    r = torch.zeros(4, 4)
    with pytest.raises(NotImplementedError):
        torch.ops.ppo_amd.gae(r, r, torch.zeros(4, 4, dtype=torch.uint8), None, 0.99, 0.95)
    with pytest.raises(NotImplementedError):
        torch.ops.ppo_amd.normalize_advantages(r, 1e-8)
