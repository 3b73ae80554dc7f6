"""PPO on vectorised CartPole-v1, every step of the loop on the GPU.

The reference trains one gymnasium CartPole-v1 episode at a time in Python
(rl/deep/runner.py:13-24 train(), :44-87 _run_episode, with PPOAgent,
rl/deep/agents/ppo.py).  Here N environments advance together: CartPoleVec
steps them in one launch, VecPPO.act samples every action in one launch into
the [T,N] rollout buffer, and VecPPO.update runs GAE + normalisation and the
epochs of minibatch updates (fused MLP kernel + clip + Adam, replayed from
graphs).  The host only draws the minibatch permutations and reads the
episode statistics once per iteration.

    python -m ppo_amd.train_cartpole [--envs 64] [--steps 128] [--iterations 50]
"""

from __future__ import annotations

import argparse
import json
import time
from typing import Callable, Optional

import torch

from .agent import MLP, PPOConfig
from .env import CartPoleVec
from .rollout import RolloutBuffer, VecPPO


def train(num_envs: int = 64, steps: int = 128, iterations: int = 50, seed: int = 24,
          hidden: int = 64, activation: str = "tanh", batch_size: int = 256,
          lr: float = 3e-4, graphs: bool = True, device: str = "cuda",
          log: Optional[Callable[[dict], None]] = None) -> list:
    """Run `iterations` of (collect `steps` x `num_envs` transitions, update)
    and return one record per iteration: completed episodes and their mean
    return, environment steps so far, seconds."""
    dev = torch.device(device)
    torch.manual_seed(seed)
    policy = MLP(4, hidden, 2, activation).to(dev)
    value = MLP(4, hidden, 1, activation).to(dev)
    env = CartPoleVec(num_envs, dev, seed=seed)
    buf = RolloutBuffer(steps, num_envs, (4,), device=dev)
    vec = VecPPO(policy, value, PPOConfig(), lr=lr, batch_size=batch_size,
                 generator=torch.Generator().manual_seed(seed), graphs=graphs)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    obs = env.reset().clone()
    records = []
    t0 = time.perf_counter()
    for it in range(iterations):
        obs = vec.collect(env, buf, obs, generator=gen)
        vec.update(buf)
        episodes, mean_return = env.episode_stats()
        rec = {"iteration": it, "episodes": episodes, "mean_return": mean_return,
               "env_steps": (it + 1) * steps * num_envs,
               "seconds": round(time.perf_counter() - t0, 3)}
        records.append(rec)
        if log is not None:
            log(rec)
    return records


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--envs", type=int, default=64)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--iterations", type=int, default=50)
    ap.add_argument("--seed", type=int, default=24)
    ap.add_argument("--hidden", type=int, default=64)
    ap.add_argument("--activation", default="tanh", choices=["tanh", "relu"])
    ap.add_argument("--batch-size", type=int, default=256)
    ap.add_argument("--lr", type=float, default=3e-4)
    ap.add_argument("--no-graphs", action="store_true")
    a = ap.parse_args()
    train(a.envs, a.steps, a.iterations, a.seed, a.hidden, a.activation, a.batch_size, a.lr,
          not a.no_graphs, log=lambda r: print(json.dumps(r), flush=True))


if __name__ == "__main__":
    main()
