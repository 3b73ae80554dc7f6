"""Writes the small golden fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

* reference_kat.json — the reference's own known-answer test, copied as data
  from rl/deep/tests/test_ppo.py:34-44 (gamma=0.8, lambda=0.5, rewards [1, 3],
  terminated [False, True], values [0.5, 1.0] -> advantages [2.1, 2.0]).
* gae_small.npz, loss_cat_small.npz, loss_gauss_small.npz — seeded inputs and
  the CPU oracle's outputs (oracle/ppo_oracle.py, itself pinned by
  tests/test_oracle.py), frozen so that later changes to the oracle or the
  kernels are caught against fixed numbers.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import ppo_oracle as ref  # noqa: E402


def main() -> None:
    with open(os.path.join(HERE, "reference_kat.json"), "w") as f:
        json.dump(
            {
                "source": "rl/deep/tests/test_ppo.py:34-44",
                "gamma": 0.8,
                "gae_lambda": 0.5,
                "rewards": [1.0, 3.0],
                "terminated": [False, True],
                "truncated": [False, False],
                "values": [0.5, 1.0],
                "advantages": [2.1, 2.0],
            },
            f,
            indent=1,
        )

    g = torch.Generator().manual_seed(24)
    T, N = 48, 12
    r = torch.randn(T, N, generator=g).numpy()
    v = torch.randn(T, N, generator=g).numpy()
    d = (torch.rand(T, N, generator=g) < 0.05).to(torch.uint8).numpy()
    lv = torch.randn(N, generator=g).numpy()
    adv, ret = ref.gae_numpy(r, v, d, lv, 0.99, 0.95)
    adv_n = ref.normalize_reference(torch.from_numpy(adv).reshape(-1)).reshape(T, N).numpy()
    np.savez(os.path.join(HERE, "gae_small.npz"), rewards=r, values=v, dones=d,
             last_value=lv, gamma=0.99, lam=0.95, adv=adv, ret=ret, adv_norm=adv_n)

    B, A = 64, 18
    logits = torch.randn(B, A, generator=g)
    old_logits = logits + 0.05 * torch.randn(B, A, generator=g)
    actions = torch.multinomial(torch.softmax(old_logits, -1), 1, generator=g).squeeze(1)
    old_lp = torch.log_softmax(old_logits, -1).gather(1, actions[:, None]).squeeze(1)
    adv_b = torch.randn(B, generator=g)
    ret_b = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    val = old_v + 0.1 * torch.randn(B, generator=g)
    o = ref.loss_categorical_reference(logits, actions, old_lp, adv_b, ret_b, val, old_v,
                                       0.2, 0.2, 0.5, 0.01)
    np.savez(os.path.join(HERE, "loss_cat_small.npz"), logits=logits.numpy(),
             actions=actions.to(torch.int32).numpy(), old_log_probs=old_lp.numpy(),
             advantages=adv_b.numpy(), returns=ret_b.numpy(), values=val.numpy(),
             old_values=old_v.numpy(), clip_ratio=0.2, vf_clip=0.2, value_coef=0.5,
             entropy_coef=0.01,
             scalars=np.array([o[k].item() for k in
                               ("loss", "policy", "value", "entropy", "approx_kl", "clipfrac")],
                              dtype=np.float32),
             dlogits=o["dlogits"].numpy(), dvalues=o["dvalues"].numpy())

    B, D = 64, 6
    mu = torch.randn(B, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0
    mu_old = mu + 0.05 * torch.randn(B, D, generator=g)
    acts = mu_old + log_std.exp() * torch.randn(B, D, generator=g)
    old_lp = torch.distributions.Normal(mu_old, log_std.exp()).log_prob(acts).sum(-1)
    adv_b = torch.randn(B, generator=g)
    ret_b = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    val = old_v + 0.1 * torch.randn(B, generator=g)
    o = ref.loss_gaussian_reference(mu, log_std, acts, old_lp, adv_b, ret_b, val, old_v,
                                    0.2, 0.2, 0.5, 0.01)
    np.savez(os.path.join(HERE, "loss_gauss_small.npz"), mu=mu.numpy(),
             log_std=log_std.numpy(), actions=acts.numpy(), old_log_probs=old_lp.numpy(),
             advantages=adv_b.numpy(), returns=ret_b.numpy(), values=val.numpy(),
             old_values=old_v.numpy(), clip_ratio=0.2, vf_clip=0.2, value_coef=0.5,
             entropy_coef=0.01,
             scalars=np.array([o[k].item() for k in
                               ("loss", "policy", "value", "entropy", "approx_kl", "clipfrac")],
                              dtype=np.float32),
             dmu=o["dmu"].numpy(), dlog_std=o["dlog_std"].numpy(), dvalues=o["dvalues"].numpy())


if __name__ == "__main__":
    main()
