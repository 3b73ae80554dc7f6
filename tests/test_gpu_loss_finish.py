"""The Gaussian loss kernels finish in-kernel: every workgroup tags its partial
sums with a hash of a call counter kept in the workspace header, and
collector workgroups sum the partials once every tag of the call is present
(csrc/loss.hip, loss_publish).  These tests call ppo_loss_gauss_f32 through the
C ABI and check what that scheme must guarantee:

* calls in a row on one workspace (growing and shrinking grids, so stale tags
  and partials of other layouts lie in the slots) give bit-identical results to
  calls on a fresh workspace;
* a workspace full of random bytes, header included, gives the same results
  (the ABI says workspace contents on entry do not matter);
* a captured graph replayed several times, with new inputs copied in and eager
  calls on the same workspace in between, matches an eager call on every
  replay (the counter lives on the device, so every replay gets a new tag).

Parity with the reference itself is covered by test_gpu_loss.py; here the
reference is the same entry point on a fresh zeroed workspace."""

import ctypes

import pytest
import torch

from ppo_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return _lib.load()


def _inputs(dev, B, D, seed):
    g = torch.Generator().manual_seed(seed)
    mu = torch.randn(B, D, generator=g)
    log_std = torch.rand(D, generator=g) - 1.0
    acts = mu + 0.05 * torch.randn(B, D, generator=g) + log_std.exp() * torch.randn(
        B, D, generator=g)
    old_lp = torch.distributions.Normal(mu, log_std.exp()).log_prob(acts).sum(-1)
    adv = torch.randn(B, generator=g)
    ret = torch.randn(B, generator=g)
    old_v = torch.randn(B, generator=g)
    v = old_v + 0.1 * torch.randn(B, generator=g)
    return [t.contiguous().to(dev) for t in (mu, log_std, acts, old_lp, adv, ret, v, old_v)]


class _Call:
    """Preallocated arguments of one ppo_loss_gauss_f32 shape."""

    def __init__(self, lib, dev, B, D, seed):
        self.lib, self.dev, self.B, self.D = lib, dev, B, D
        self.x = _inputs(dev, B, D, seed)
        self.dmu = torch.empty(B, D, device=dev)
        self.dls = torch.empty(D, device=dev)
        self.dv = torch.empty(B, device=dev)
        self.sc = torch.empty(_lib.PPO_NUM_SCALARS, device=dev)
        self.params = _lib.LossParams(0.2, 0.2, 0.5, 0.01)
        self.nbytes = lib.ppo_loss_gauss_workspace_bytes(B, D)

    def run(self, ws):
        mu, ls, acts, old_lp, adv, ret, v, old_v = self.x
        stream = torch.cuda.current_stream(self.dev).cuda_stream
        code = self.lib.ppo_loss_gauss_f32(
            mu.data_ptr(), ls.data_ptr(), self.B, self.D, acts.data_ptr(), old_lp.data_ptr(),
            adv.data_ptr(), ret.data_ptr(), v.data_ptr(), old_v.data_ptr(),
            ctypes.byref(self.params), self.dmu.data_ptr(), self.dls.data_ptr(),
            self.dv.data_ptr(), self.sc.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check("ppo_loss_gauss_f32", code)

    def outputs(self):
        return [t.detach().cpu().clone() for t in (self.sc, self.dls, self.dmu, self.dv)]

    def fresh(self):
        """Outputs of a call on a new zeroed workspace."""
        ws = torch.zeros(self.nbytes, dtype=torch.uint8, device=self.dev)
        self.run(ws)
        torch.cuda.synchronize(self.dev)
        return self.outputs()


def _assert_same(got, want, what):
    for g, w, name in zip(got, want, ("scalars", "dlog_std", "dmu", "dvalues")):
        assert torch.isfinite(g).all(), (what, name)
        assert torch.equal(g, w), (what, name, g, w)


def test_calls_in_a_row_on_one_workspace(lib):
    dev = torch.device("cuda:0")
    # grids: many workgroups, one, a few (D > grid: workgroups take several
    # column groups), many again, and several calls of one shape
    shapes = [(600_000, 6, 1), (40, 6, 2), (700, 24, 3), (300_000, 8, 4), (300_000, 8, 5),
              (300_000, 8, 6), (2_000, 1, 7)]
    calls = [_Call(lib, dev, B, D, seed) for B, D, seed in shapes]
    ws = torch.zeros(max(c.nbytes for c in calls), dtype=torch.uint8, device=dev)
    for c in calls:
        print(f"loss_gauss in a row B={c.B} D={c.D}", flush=True)
        want = c.fresh()
        c.run(ws)
        torch.cuda.synchronize(dev)
        _assert_same(c.outputs(), want, (c.B, c.D))


@pytest.mark.parametrize("B,D", [(500_000, 6), (1_000, 17), (3, 2)])
def test_workspace_of_random_bytes(lib, B, D):
    dev = torch.device("cuda:0")
    print(f"loss_gauss random workspace B={B} D={D}", flush=True)
    c = _Call(lib, dev, B, D, seed=B + D)
    want = c.fresh()
    g = torch.Generator(device=dev).manual_seed(B)
    ws = torch.randint(0, 256, (c.nbytes,), dtype=torch.uint8, device=dev, generator=g)
    c.run(ws)
    torch.cuda.synchronize(dev)
    _assert_same(c.outputs(), want, "random workspace")


def test_graph_replays_match_eager(lib):
    dev = torch.device("cuda:0")
    B, D = 200_000, 6
    print(f"loss_gauss graph replays B={B} D={D}", flush=True)
    c = _Call(lib, dev, B, D, seed=5)
    ws = torch.zeros(c.nbytes, dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream(dev)
    c.run(ws)  # warm-up before capture
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        c.run(ws)
    for rep in range(4):
        new = _inputs(dev, B, D, seed=100 + rep)
        for dst, src in zip(c.x, new):
            dst.copy_(src)
        ref = _Call(lib, dev, B, D, seed=100 + rep)
        want = ref.fresh()
        graph.replay()
        torch.cuda.synchronize(dev)
        _assert_same(c.outputs(), want, f"replay {rep}")
        # an eager call on the same workspace between replays
        c.run(ws)
        torch.cuda.synchronize(dev)
        _assert_same(c.outputs(), want, f"eager after replay {rep}")
