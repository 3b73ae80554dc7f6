"""Graph-replayed update loop: VecPPO(graphs=True) and a captured
ClippedAdam(capturable=True) step against the same work run eagerly.

Every graph is replayed several times with eager work (rollout writes, GAE,
host synchronisation) between the replays, and every replay's result is
checked.  The graph path runs the same kernels on the same data as the eager
fused path; the only difference is where Adam's bias corrections are formed
(on the device from the step counter instead of on the host), which can move
a parameter by an ulp, so parameters are compared at rel 1e-5 / abs 1e-7.
"""

import copy

import pytest
import torch

import ppo_amd
from ppo_amd.agent import MLP, PPOConfig

pytestmark = pytest.mark.gpu


def _fill(buf, T, N, seed, dev, D=None):
    g = torch.Generator().manual_seed(seed)
    buf.reset()
    for _ in range(T):
        obs = torch.randn(N, 4, generator=g)
        if D is None:
            act = torch.randint(0, 3, (N,), generator=g, dtype=torch.int32)
        else:
            act = torch.randn(N, D, generator=g)
        buf.add(obs.to(dev), act.to(dev), torch.randn(N, generator=g).to(dev),
                (torch.rand(N, generator=g) < 0.05).to(torch.uint8).to(dev),
                torch.randn(N, generator=g).to(dev), (torch.randn(N, generator=g) - 1).to(dev))
    buf.finish(torch.randn(N, generator=g).to(dev))


def _agents(dev, graph_chunk, D=None, vf_clip=None):
    torch.manual_seed(11)
    out = D or 3
    policy, value = MLP(4, 32, out, "tanh").to(dev), MLP(4, 32, 1, "tanh").to(dev)
    log_std = torch.nn.Parameter(torch.full((D,), -0.3, device=dev)) if D else None
    cfg = PPOConfig(epochs=3, vf_clip=vf_clip)
    made = []
    for graphs in (False, True):
        p, v = copy.deepcopy(policy), copy.deepcopy(value)
        ls = torch.nn.Parameter(log_std.detach().clone()) if D else None
        made.append(ppo_amd.VecPPO(p, v, cfg, lr=1e-3, batch_size=48, log_std=ls,
                                   generator=torch.Generator().manual_seed(3),
                                   graphs=graphs, graph_chunk=graph_chunk))
    return made


def _check(eager, graphed, s_eager, s_graph):
    for a, b in zip(graphed.parameters, eager.parameters):
        torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-5, atol=1e-7)
    for k in ("loss", "policy", "value", "entropy"):
        torch.testing.assert_close(s_graph[k], s_eager[k], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("graph_chunk", [64, 2])
def test_vecppo_graphs_match_eager_categorical(dev, graph_chunk):
    T, N = 20, 10  # 200 samples: 4 minibatches of 48 and one of 8
    eager, graphed = _agents(dev, graph_chunk, vf_clip=0.2)
    bufs = [ppo_amd.RolloutBuffer(T, N, (4,), device=dev) for _ in range(2)]
    for it in range(3):
        for b in bufs:
            _fill(b, T, N, 100 + it, dev)
        s_e = eager.update(bufs[0])
        s_g = graphed.update(bufs[1])
        torch.cuda.synchronize()
        assert graphed.update_graphed_ready()
        _check(eager, graphed, s_e, s_g)
    # one graph sequence per epoch, each of ceil(5 minibatches / chunk) graphs
    assert len(graphed._plan.graphs) == 3
    assert all(len(seq) == -(-5 // graph_chunk) for seq in graphed._plan.graphs)
    assert graphed.optimizer.step_count() == 3 * 3 * 5


def test_vecppo_graphs_match_eager_gaussian(dev):
    T, N, D = 16, 12, 3
    eager, graphed = _agents(dev, 64, D=D)
    bufs = [ppo_amd.RolloutBuffer(T, N, (4,), device=dev, action_dim=D) for _ in range(2)]
    for it in range(3):
        for b in bufs:
            _fill(b, T, N, 200 + it, dev, D=D)
        s_e = eager.update(bufs[0])
        s_g = graphed.update(bufs[1])
        torch.cuda.synchronize()
        _check(eager, graphed, s_e, s_g)


def test_vecppo_graphs_recapture_on_new_shape(dev):
    eager, graphed = _agents(dev, 64)
    for T in (20, 12, 20):
        bufs = [ppo_amd.RolloutBuffer(T, 10, (4,), device=dev) for _ in range(2)]
        for b in bufs:
            _fill(b, T, 10, 300 + T, dev)
        s_e = eager.update(bufs[0])
        s_g = graphed.update(bufs[1])
        torch.cuda.synchronize()
        _check(eager, graphed, s_e, s_g)


def test_clipped_adam_step_in_graph_replays(dev):
    shapes = [(33, 7), (7,), (5000,)]
    g = torch.Generator().manual_seed(9)
    init = [torch.randn(*s, generator=g).to(dev) for s in shapes]
    p_ref = [x.clone().requires_grad_(True) for x in init]
    p_got = [x.clone().requires_grad_(True) for x in init]
    opt_ref = torch.optim.Adam(p_ref, lr=1e-2)
    opt_got = ppo_amd.ClippedAdam(p_got, lr=1e-2, max_grad_norm=0.5, capturable=True)
    static_g = [torch.zeros_like(x) for x in init]
    for p, sg in zip(p_got, static_g):
        p.grad = sg
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        opt_got.step()  # eager warm-up step 1 (all-zero gradients)
    torch.cuda.current_stream().wait_stream(s)
    for p in p_ref:
        p.grad = torch.zeros_like(p)
    opt_ref.step()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        norm = opt_got.step()
    for step in range(4):
        grads = [torch.randn(*x.shape, generator=g).to(dev) * (1 + step) for x in init]
        for sg, gr in zip(static_g, grads):
            sg.copy_(gr)
        for p, gr in zip(p_ref, grads):
            p.grad = gr.clone()
        norm_ref = torch.nn.utils.clip_grad_norm_(p_ref, 0.5)
        opt_ref.step()
        graph.replay()
        torch.cuda.synchronize()
        assert norm.item() == pytest.approx(norm_ref.item(), rel=1e-6)
        for a, b in zip(p_got, p_ref):
            torch.testing.assert_close(a.detach(), b.detach(), rtol=2e-6, atol=1e-7)
    assert opt_got.step_count() == 5
