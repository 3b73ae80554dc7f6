"""GPU parity of the GAE kernels (ppo_gae_f32 / ppo_gae_norm_f32) against the
CPU oracle (oracle/gae_ref.c: the reference recurrence, ppo.py:173-193, in
fp64 with the reference's operation order).

Tolerance: the kernel evaluates the same fp64 recurrence in the same order;
only the carries entering each thread's segment are composed with a scan
(reassociated fp64), so outputs may differ from the oracle by at most one
fp32 ulp, or by 1e-9 absolute where the fp32 result is a near-cancellation.
The benchmark's stated bar (rel 1e-5) is far looser.  Returns = advantages + values must
then match bit for bit wherever the advantages do.
"""

import json
import os

import numpy as np
import pytest
import torch

import ppo_amd
from oracle import ppo_oracle as ref

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _c_oracle():
    ref.build_c()


@pytest.fixture
def no_resident(monkeypatch):
    """Turns the resident pass off, so shapes it would take run on the strip
    walk / span / tile passes they are chosen to exercise."""
    monkeypatch.setenv("PPO_AMD_GAE_RESIDENT", "0")


def _inputs(T, N, p_done, seed, last=True):
    g = torch.Generator().manual_seed(seed)
    r = torch.randn(T, N, generator=g)
    v = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < p_done).to(torch.uint8)
    lv = torch.randn(N, generator=g) if last else None
    return r, v, d, lv


def assert_gae_close(adv, adv_ref):
    adv = np.asarray(adv, dtype=np.float32)
    adv_ref = np.asarray(adv_ref, dtype=np.float32)
    assert adv.shape == adv_ref.shape
    ulp = np.abs(adv.view(np.int32).astype(np.int64) - adv_ref.view(np.int32).astype(np.int64))
    absdiff = np.abs(adv.astype(np.float64) - adv_ref.astype(np.float64))
    bad = (ulp > 1) & (absdiff > 1e-9)
    assert not bad.any(), (
        f"{int(bad.sum())} elements off by >1 ulp; worst abs {absdiff.max():.3e} "
        f"at {np.unravel_index(absdiff.argmax(), absdiff.shape)}"
    )
    return float((ulp == 0).mean())


def _run(dev, T, N, p, seed, gamma=0.99, lam=0.95, last=True):
    r, v, d, lv = _inputs(T, N, p, seed, last)
    print(f"gae T={T} N={N} p={p} seed={seed} last={last}", flush=True)
    adv, ret = ppo_amd.gae(r.to(dev), v.to(dev), d.to(dev),
                           None if lv is None else lv.to(dev), gamma, lam)
    a_ref, r_ref = ref.gae_c(r.numpy(), v.numpy(), d.numpy(),
                             None if lv is None else lv.numpy(), gamma, lam)
    exact = assert_gae_close(adv.cpu().numpy(), a_ref)
    # returns are the fp32 sum of the (checked) advantages and the values
    np.testing.assert_array_equal(ret.cpu().numpy(), adv.cpu().numpy() + v.numpy())
    return exact


def test_reference_known_answer_n1(dev):
    """rl/deep/tests/test_ppo.py:34-44 through the GPU kernel."""
    with open(os.path.join(GOLDEN, "reference_kat.json")) as f:
        kat = json.load(f)
    r = torch.tensor(kat["rewards"], device=dev)
    v = torch.tensor(kat["values"], device=dev)
    d = torch.tensor([a or b for a, b in zip(kat["terminated"], kat["truncated"])],
                     dtype=torch.bool, device=dev)
    adv, ret = ppo_amd.gae(r, v, d, None, kat["gamma"], kat["gae_lambda"])
    assert adv.cpu().tolist() == pytest.approx(kat["advantages"])
    a_ref = ref.advantages_python(kat["rewards"], d.cpu().tolist(), kat["values"],
                                  kat["gamma"], kat["gae_lambda"])
    np.testing.assert_array_equal(adv.cpu().numpy(), np.array(a_ref, np.float32))


def test_golden_fixture(dev):
    z = np.load(os.path.join(GOLDEN, "gae_small.npz"))
    t = lambda k: torch.from_numpy(z[k]).to(dev)  # noqa: E731
    adv, ret, adv_n = ppo_amd.gae_normalize(t("rewards"), t("values"), t("dones"),
                                            t("last_value"), float(z["gamma"]), float(z["lam"]))
    np.testing.assert_array_equal(adv.cpu().numpy(), z["adv"])
    np.testing.assert_array_equal(ret.cpu().numpy(), z["ret"])
    np.testing.assert_allclose(adv_n.cpu().numpy(), z["adv_norm"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize(
    "T,N,p",
    [
        (1, 1, 0.0), (1, 1, 1.0), (2, 1, 0.0), (5, 1, 0.2), (300, 1, 0.01),
        (5000, 1, 0.001),                     # N=1 across several tiles (scalar path)
        (37, 3, 0.1), (129, 7, 0.05),         # N not a multiple of 4
        (1, 4, 0.0), (33, 4, 0.1), (100, 8, 0.05), (128, 8, 0.005),
        (64, 12, 0.3), (513, 16, 0.01), (2000, 16, 0.001),
        (7, 260, 0.1), (65, 1028, 0.02), (257, 4096, 0.01),
    ],
)
def test_gae_matches_oracle(dev, T, N, p):
    _run(dev, T, N, p, seed=T * 7919 + N)


@pytest.mark.parametrize("p", [0.0, 1.0])
def test_gae_all_or_no_dones(dev, p):
    _run(dev, 700, 20, p, seed=3)


def test_gae_without_bootstrap(dev):
    _run(dev, 1000, 12, 0.01, seed=4, last=False)


def test_gae_misaligned_buffers(dev):
    """Views that start one element into an allocation are not 16-byte
    aligned: the kernel must take its scalar path and still agree."""
    T, N = 300, 8
    r, v, d, lv = _inputs(T, N, 0.05, seed=9)
    rb = torch.empty(T * N + 1, device=dev)
    vb = torch.empty(T * N + 1, device=dev)
    db = torch.empty(T * N + 1, dtype=torch.uint8, device=dev)
    rb[1:] = r.reshape(-1).to(dev)
    vb[1:] = v.reshape(-1).to(dev)
    db[1:] = d.reshape(-1).to(dev)
    adv, ret = ppo_amd.gae(rb[1:].view(T, N), vb[1:].view(T, N), db[1:].view(T, N),
                           lv.to(dev), 0.99, 0.95)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    assert_gae_close(adv.cpu().numpy(), a_ref)


def test_gae_nonzero_done_bytes_count_as_done(dev):
    T, N = 50, 4
    r, v, d, lv = _inputs(T, N, 0.2, seed=10)
    d2 = d * torch.randint(1, 255, (T, N), dtype=torch.uint8)
    a1, _ = ppo_amd.gae(r.to(dev), v.to(dev), d.to(dev), lv.to(dev))
    a2, _ = ppo_amd.gae(r.to(dev), v.to(dev), d2.to(dev), lv.to(dev))
    torch.testing.assert_close(a1, a2, rtol=0, atol=0)


def test_gae_config2_full_size(dev):
    """Configuration 2: T=2048, N=4096, dones Bernoulli(0.01)."""
    exact = _run(dev, 2048, 4096, 0.01, seed=24)
    assert exact > 0.99


def test_gae_config3_full_size(dev):
    """Configuration 3: T=1,048,576, N=16, dones Bernoulli(0.001), gamma .999."""
    exact = _run(dev, 1_048_576, 16, 0.001, seed=24, gamma=0.999, lam=0.95)
    assert exact > 0.99


def test_gae_normalize_over_2_30_elements(dev):
    """T = N = 32768 (2^30 elements, ~25 GB on the device): the strip walk
    declines (its offsets are 32-bit) and the span passes run with 64-bit
    offsets.  Inputs are drawn on the device; 16 env columns (env columns are
    independent) are checked against the C oracle to the usual ulp bar, the
    returns bit-exactly, the normaliser's mean/std against an fp64 reduction
    of the advantages (relative 1e-6) and adv_n bit-exactly against the fp32
    formula at the returned statistics."""
    T = N = 32768
    print(f"gae_normalize T={T} N={N}", flush=True)
    g = torch.Generator(device=dev).manual_seed(77)
    r = torch.randn(T, N, device=dev, generator=g)
    v = torch.randn(T, N, device=dev, generator=g)
    d = (torch.rand(T, N, device=dev, generator=g) < 0.01).to(torch.uint8)
    lv = torch.randn(N, device=dev, generator=g)
    adv, ret, adv_n, stats = ppo_amd.gae_normalize(r, v, d, lv, 0.99, 0.95, return_stats=True)
    cols = torch.tensor([0, 1, 5, 1023, 4096, 9999, 16383, 16384, 20000, 24575, 30001, 32000,
                         32764, 32765, 32766, 32767], device=dev)
    rc, vc, dc = (x.index_select(1, cols).cpu().numpy() for x in (r, v, d))
    a_ref, _ = ref.gae_c(rc, vc, dc, lv.index_select(0, cols).cpu().numpy(), 0.99, 0.95)
    a_got = adv.index_select(1, cols)
    exact = assert_gae_close(a_got.cpu().numpy(), a_ref)
    assert exact > 0.99
    assert torch.equal(ret.index_select(1, cols), a_got + v.index_select(1, cols))
    s1 = s2 = 0.0
    for k in range(0, T, 4096):  # fp64 moments in slices (an fp64 copy would be 8 GB)
        x = adv[k:k + 4096].double()
        s1 += float(x.sum())
        s2 += float((x * x).sum())
    n = float(T * N)
    mean = s1 / n
    std = ((s2 - s1 * mean) / (n - 1)) ** 0.5
    assert stats[0].item() == pytest.approx(mean, rel=1e-6, abs=1e-7)
    assert stats[1].item() == pytest.approx(std, rel=1e-6)
    want_n = (a_got - stats[0]) / (stats[1] + torch.tensor(1e-8, device=dev))
    assert torch.equal(adv_n.index_select(1, cols), want_n)


def test_gae_multi_round_chunk_fold(dev):
    """T=262144, N=64: 4096 tiles in 32 carry chunks, more than one block's
    rows, so the later-chunk fold takes two rounds."""
    exact = _run(dev, 262_144, 64, 0.002, seed=31, gamma=0.997, lam=0.97)
    assert exact > 0.99


def test_gae_repeatable(dev):
    r, v, d, lv = _inputs(1024, 64, 0.01, seed=12)
    args = (r.to(dev), v.to(dev), d.to(dev), lv.to(dev))
    a1, _, n1 = ppo_amd.gae_normalize(*args)
    a2, _, n2 = ppo_amd.gae_normalize(*args)
    assert torch.equal(a1, a2) and torch.equal(n1, n2)


# ---------------------------------------------------------------------------
# REINFORCE returns (rl/deep/agents/reinforce.py:57-66) through the GAE kernel
# ---------------------------------------------------------------------------
def _reinforce_python(rewards, gamma):
    """reinforce.py:57-63 restated: value = reward + gamma * value."""
    returns = []
    value = 0.0
    for reward in reversed(rewards):
        value = reward + gamma * value
        returns.append(value)
    returns.reverse()
    return returns


@pytest.mark.parametrize("T", [1, 2, 37, 500, 5000])
def test_discounted_returns_bit_identical_to_reference_loop(dev, T):
    g = torch.Generator().manual_seed(T)
    r = torch.randn(T, generator=g)
    got = ppo_amd.discounted_returns(r.to(dev), gamma=0.97).cpu().numpy()
    expect = np.array(_reinforce_python([float(x) for x in r], 0.97), dtype=np.float32)
    np.testing.assert_array_equal(got, expect)
    centered = ppo_amd.discounted_returns(r.to(dev), gamma=0.97, center=True).cpu()
    ref_t = torch.as_tensor(expect)
    torch.testing.assert_close(centered, ref_t - ref_t.mean(), rtol=1e-6, atol=1e-6)


def test_discounted_returns_vectorised_with_dones(dev):
    T, N = 3000, 20
    g = torch.Generator().manual_seed(2)
    r = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.01).to(torch.uint8)
    boot = torch.randn(N, generator=g)
    got = ppo_amd.discounted_returns(r.to(dev), d.to(dev), 0.99, boot.to(dev)).cpu().numpy()
    # oracle: GAE with lambda = 1 and zero values
    expect, _ = ref.gae_c(r.numpy(), np.zeros((T, N), np.float32), d.numpy(), boot.numpy(),
                          0.99, 1.0)
    assert_gae_close(got, expect)
    # per env it is the reference loop restarted after each done
    for n in range(3):
        col, start = [], 0
        ends = list(np.nonzero(d[:, n].numpy())[0]) + [T - 1]
        for e in ends:
            seg = [float(x) for x in r[start:e + 1, n]]
            if e == T - 1 and not d[T - 1, n]:
                vals = []
                v = float(boot[n])
                for x in reversed(seg):
                    v = x + 0.99 * v
                    vals.append(v)
                col += list(reversed(vals))
            else:
                col += _reinforce_python(seg, 0.99)
            start = e + 1
            if start >= T:
                break
        np.testing.assert_allclose(got[:len(col), n], np.array(col, np.float32), rtol=1e-6,
                                   atol=1e-6)


# ---------------------------------------------------------------------------
# Strip walk (wide rollouts, N >= 2048 aligned): one workgroup per strip of
# 8/16/32 envs walks the horizon backwards in chunks of 1024/512/256 steps.
# Shapes cover each strip width, horizons shorter than, equal to and not a
# multiple of a chunk, odd and even chunk counts, a partial last strip (N not
# a multiple of the strip width), and short horizons that stay on the tile
# passes (T < a quarter of a chunk).
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "T,N,p",
    [
        (1, 2048, 0.1), (3, 4096, 0.1), (100, 2048, 0.02),    # tile passes
        (300, 2048, 0.02), (1024, 2048, 0.01), (2048, 2048, 0.01),  # E=8: <1, 1, 2 chunks
        (1500, 2052, 0.01),                                    # E=8, partial strip
        (200, 4096, 0.01), (512, 4096, 0.01), (1536, 4096, 0.01),  # E=16: <1, 1, 3 chunks
        (1000, 4100, 0.02),                                    # E=16, partial strip
        (129, 8192, 0.05), (640, 8196, 0.01),                  # E=32
    ],
)
def test_gae_strip_walk_matches_oracle(no_resident, dev, T, N, p):
    exact = _run(dev, T, N, p, seed=T * 31 + N)
    assert exact > 0.99


def test_gae_strip_walk_without_bootstrap(no_resident, dev):
    _run(dev, 700, 4096, 0.01, seed=41, last=False)


def test_gae_strip_walk_all_or_no_dones(no_resident, dev):
    _run(dev, 300, 2048, 1.0, seed=42)
    _run(dev, 300, 2048, 0.0, seed=43)


def test_discounted_returns_strip_walk(no_resident, dev):
    """values = None (REINFORCE returns) on the strip walk."""
    T, N = 600, 4096
    g = torch.Generator().manual_seed(44)
    r = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.01).to(torch.uint8)
    boot = torch.randn(N, generator=g)
    got = ppo_amd.discounted_returns(r.to(dev), d.to(dev), 0.99, boot.to(dev)).cpu().numpy()
    expect, _ = ref.gae_c(r.numpy(), np.zeros((T, N), np.float32), d.numpy(), boot.numpy(),
                          0.99, 1.0)
    assert_gae_close(got, expect)


def test_gae_normalize_strip_walk_matches_separate_ops(no_resident, dev):
    g = torch.Generator().manual_seed(45)
    T, N = 777, 2056
    r = torch.randn(T, N, generator=g).to(dev)
    v = torch.randn(T, N, generator=g).to(dev)
    d = (torch.rand(T, N, generator=g) < 0.02).to(torch.uint8).to(dev)
    lv = torch.randn(N, generator=g).to(dev)
    adv, ret, adv_n = ppo_amd.gae_normalize(r, v, d, lv)
    adv2, ret2 = ppo_amd.gae(r, v, d, lv)
    assert torch.equal(adv, adv2) and torch.equal(ret, ret2)
    torch.testing.assert_close(adv_n, ppo_amd.normalize_advantages(adv2), rtol=1e-6, atol=1e-7)
    n_ref = ref.normalize_reference(adv2.cpu().reshape(-1)).reshape(T, N)
    torch.testing.assert_close(adv_n.cpu(), n_ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# Span passes (aligned rollouts narrower than the strip walk): strips of
# E = 4..64 envs, 4096-element tiles, spans of tiles composed right to left.
# ---------------------------------------------------------------------------
def _gae_abi(dev, r, v, d, lv, gamma, lam, norm=False, fill=0xAB):
    """ppo_gae_f32 / ppo_gae_norm_f32 through the C ABI with a fresh workspace
    filled with `fill` (its contents on entry must not matter)."""
    from ppo_amd import _lib

    lib = _lib.load()
    T, N = r.shape
    ws = torch.full((lib.ppo_gae_workspace_bytes(T, N),), fill, dtype=torch.uint8, device=dev)
    adv, ret, adv_n = (torch.empty(T, N, device=dev) for _ in range(3))
    stream = torch.cuda.current_stream(dev).cuda_stream
    lvp = None if lv is None else lv.data_ptr()
    if norm:
        rc = lib.ppo_gae_norm_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lvp, T, N, gamma, lam,
                                  1e-8, adv.data_ptr(), ret.data_ptr(), adv_n.data_ptr(), None,
                                  ws.data_ptr(), ws.numel(), stream)
    else:
        rc = lib.ppo_gae_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lvp, T, N, gamma, lam,
                             adv.data_ptr(), ret.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    assert rc == 0
    torch.cuda.synchronize(dev)
    return adv, ret, adv_n


@pytest.mark.parametrize(
    "T,N,p",
    [
        (4096, 4, 0.01),     # E=4: 1024-step tiles, one strip
        (1500, 8, 0.02),     # E=8, partial last tile
        (10_000, 16, 0.005), # E=16 (config 3's geometry), 40 tiles
        (3000, 32, 0.01),    # E=32
        (777, 96, 0.05),     # E=32, three strips
        (4000, 64, 0.001),   # E=64
        (129, 1984, 0.02),   # E=64, 31 strips, partial tiles
        (50, 1020, 0.1),     # E=4, 255 strips, one short tile each
        (1, 16, 0.0),        # one step
        (3_000_000, 4, 0.0005),  # spans of many tiles
        (1 << 20, 16, 0.001),    # config 3's shape without the normaliser
    ],
)
def test_gae_span_matches_oracle(no_resident, dev, T, N, p):
    """With the normaliser every aligned rollout narrower than the strip walk
    takes the span passes; without it the narrow (N < 64), large ones do."""
    r, v, d, lv = _inputs(T, N, p, seed=T + 31 * N)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    for norm in (True, False):
        print(f"gae span T={T} N={N} p={p} norm={norm}", flush=True)
        adv, ret, adv_n = _gae_abi(dev, r.to(dev), v.to(dev), d.to(dev), lv.to(dev), 0.99, 0.95,
                                   norm=norm)
        assert_gae_close(adv.cpu().numpy(), a_ref)
        np.testing.assert_array_equal(ret.cpu().numpy(), adv.cpu().numpy() + v.numpy())
        if norm:
            torch.testing.assert_close(adv_n, ppo_amd.normalize_advantages(adv), rtol=1e-6,
                                       atol=1e-7)


def test_gae_span_normalize_matches_separate_ops(no_resident, dev):
    T, N = 20_000, 24
    r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.01, seed=12))
    print(f"gae span norm T={T} N={N}", flush=True)
    adv, ret, adv_n = _gae_abi(dev, r, v, d, lv, 0.995, 0.9, norm=True)
    a_ref, _ = ref.gae_c(r.cpu().numpy(), v.cpu().numpy(), d.cpu().numpy(), lv.cpu().numpy(),
                         0.995, 0.9)
    assert_gae_close(adv.cpu().numpy(), a_ref)
    torch.testing.assert_close(adv_n, ppo_amd.normalize_advantages(adv), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("T,N", [(1 << 17, 16), (1 << 19, 4)])
def test_discounted_returns_span_passes(no_resident, dev, T, N):
    """REINFORCE returns (values absent) on shapes that take the span passes
    (aligned, N < 64, >= 2^20 elements): GAE with lambda = 1 and zero values."""
    g = torch.Generator().manual_seed(T + N)
    r = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.002).to(torch.uint8)
    boot = torch.randn(N, generator=g)
    print(f"discounted returns span T={T} N={N}", flush=True)
    got = ppo_amd.discounted_returns(r.to(dev), d.to(dev), 0.997, boot.to(dev)).cpu().numpy()
    expect, _ = ref.gae_c(r.numpy(), np.zeros((T, N), np.float32), d.numpy(), boot.numpy(),
                          0.997, 1.0)
    assert_gae_close(got, expect)


def test_gae_span_workspace_contents_do_not_matter(no_resident, dev):
    T, N = 65_536, 16
    r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.001, seed=13))
    outs = [_gae_abi(dev, r, v, d, lv, 0.999, 0.95, fill=f)[0] for f in (0x00, 0xFF, 0x7F)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


# ---------------------------------------------------------------------------
# Seeded sweep across the routing boundaries: shapes drawn so that the tile
# passes, the span passes and the strip walk all occur (aligned and unaligned
# N, short and long horizons), with and without the fused normaliser.
# ---------------------------------------------------------------------------
def _sweep_shapes(count=24, seed=2024, max_elems=1 << 21):
    rng = np.random.default_rng(seed)
    shapes = []
    while len(shapes) < count:
        N = int(2 ** rng.uniform(0, 13))
        if rng.random() < 0.6:
            N = max(4, N - N % 4)  # aligned: span passes / strip walk eligible
        T = int(2 ** rng.uniform(0, 20))
        T = max(1, min(T, max_elems // N))
        shapes.append((T, N, float(rng.choice([0.0, 0.001, 0.01, 0.2])), bool(rng.random() < 0.5)))
    # strip walk: 8-env strips, 32-env strips, and 16-env strips whose last
    # strip is ragged (N % 16 == 4)
    shapes += [(1024, 2048, 0.01, False), (512, 8192, 0.01, True), (2048, 4100, 0.01, True)]
    return shapes


@pytest.mark.parametrize("resident", [True, False])
@pytest.mark.parametrize("T,N,p,norm", _sweep_shapes())
def test_gae_routing_sweep_matches_oracle(dev, monkeypatch, T, N, p, norm, resident):
    if not resident:
        monkeypatch.setenv("PPO_AMD_GAE_RESIDENT", "0")
    seed = T * 31 + N * 7 + int(norm)
    r, v, d, lv = _inputs(T, N, p, seed)
    print(f"gae sweep T={T} N={N} p={p} norm={norm} seed={seed} resident={resident}", flush=True)
    args = (r.to(dev), v.to(dev), d.to(dev), lv.to(dev), 0.99, 0.95)
    if norm:
        adv, ret, adv_n = ppo_amd.gae_normalize(*args)
    else:
        adv, ret = ppo_amd.gae(*args)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    assert_gae_close(adv.cpu().numpy(), a_ref)
    np.testing.assert_array_equal(ret.cpu().numpy(), adv.cpu().numpy() + v.numpy())
    if norm:
        n_ref = ref.normalize_reference(adv.cpu().reshape(-1)).reshape(T, N)
        torch.testing.assert_close(adv_n.cpu(), n_ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# Resident pass (aligned rollouts whose tiles fit on the device at once):
# tiles of 64, 128 or 32 envs x 512-2048 steps held in registers, composites
# exchanged between the tiles of an env column, statistics between all tiles.
# Shapes cover one tile, several tiles per column (one look-back pass and
# more than one: 16 composites are read per pass at E = 32), ragged last
# tiles, each tile width, the halved segment length of short horizons, and
# the largest grid (config 2).
# ---------------------------------------------------------------------------
RESIDENT_SHAPES = [
    (2048, 4096, 0.01),   # config 2: 128-env tiles, 16 steps per thread, 32 columns x 8 tiles
    (1000, 8192, 0.01),   # 128-env tiles, ragged last tile
    (1024, 1024, 0.02),   # 4 steps per thread, 128 tiles
    (3000, 1024, 0.01),   # 8 steps per thread, ragged last tile
    (1025, 2048, 0.05),   # last tile holds one row
    (16_384, 512, 0.002), # 32 tiles in a column: a look-back of 31 composites
    (4000, 288, 0.01),    # 32-env tiles, 4 steps per thread
    (15_500, 288, 0.001), # 32-env tiles, 16 steps per thread, ragged
    (2048, 1024, 0.0),    # no dones: every carry crosses every tile
    (1024, 2048, 1.0),    # every step done
    (32_768, 144, 0.01),  # 16-env tiles (paired rows), 16 steps per thread
    (16_000, 144, 0.01),  # 16-env tiles, 8 steps per thread, ragged
    (8_000, 144, 0.02),   # 16-env tiles, 4 steps per thread, ragged
]


def _route(T, N, norm, has_values=True):
    from ppo_amd import _lib

    return _lib.GAE_ROUTES[_lib.load().ppo_gae_route(T, N, int(norm), int(has_values))]


def _resident_case(dev, T, N, p, norm, seed, last=True, fill=0xAB):
    assert _route(T, N, norm) == "resident"
    r, v, d, lv = (None if x is None else x.to(dev) for x in _inputs(T, N, p, seed, last))
    print(f"gae resident T={T} N={N} p={p} norm={norm} seed={seed} last={last} fill={fill}",
          flush=True)
    adv, ret, adv_n = _gae_abi(dev, r, v, d, lv, 0.99, 0.95, norm=norm, fill=fill)
    a_ref, _ = ref.gae_c(r.cpu().numpy(), v.cpu().numpy(), d.cpu().numpy(),
                         None if lv is None else lv.cpu().numpy(), 0.99, 0.95)
    exact = assert_gae_close(adv.cpu().numpy(), a_ref)
    assert torch.equal(ret, adv + v)
    if norm:
        n_ref = ref.normalize_reference(torch.from_numpy(a_ref).reshape(-1)).reshape(T, N)
        torch.testing.assert_close(adv_n.cpu(), n_ref, rtol=1e-5, atol=1e-6)
    return exact, adv, adv_n


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("T,N,p", RESIDENT_SHAPES)
def test_gae_resident_matches_oracle(dev, T, N, p, norm):
    exact, _, _ = _resident_case(dev, T, N, p, norm, seed=T * 13 + N)
    assert exact > 0.99


def test_gae_resident_without_bootstrap(dev):
    _resident_case(dev, 1500, 1024, 0.01, True, seed=5, last=False)


def test_gae_resident_workspace_contents_do_not_matter(dev):
    """The slots are cleared by the call itself: a workspace full of any
    pattern, or left by a previous call of another shape, gives the same
    bits."""
    outs = [_resident_case(dev, 2048, 512, 0.01, True, seed=6, fill=f)[1:]
            for f in (0x00, 0xFF, 0x7F)]
    for a, n in outs[1:]:
        assert torch.equal(a, outs[0][0]) and torch.equal(n, outs[0][1])
    # one workspace through calls of several shapes, then the first again
    from ppo_amd import _lib

    lib = _lib.load()
    shapes = [(2048, 512), (100, 64), (20_000, 32), (2048, 512)]
    nbytes = max(lib.ppo_gae_workspace_bytes(T, N) for T, N in shapes)
    ws = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    got = []
    for T, N in shapes:
        r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.01, seed=6))
        adv, ret, adv_n = (torch.empty(T, N, device=dev) for _ in range(3))
        rc = lib.ppo_gae_norm_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N,
                                  0.99, 0.95, 1e-8, adv.data_ptr(), ret.data_ptr(),
                                  adv_n.data_ptr(), None, ws.data_ptr(), ws.numel(), stream)
        assert rc == 0
        got.append((adv, adv_n))
    torch.cuda.synchronize(dev)
    assert torch.equal(got[0][0], got[3][0]) and torch.equal(got[0][1], got[3][1])
    assert torch.equal(got[0][0], outs[0][0]) and torch.equal(got[0][1], outs[0][1])


def test_gae_resident_normalise_in_place(dev):
    """adv_norm_out may alias adv_out."""
    T, N = 2048, 1024
    assert _route(T, N, True) == "resident"
    r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.01, seed=8))
    adv, ret, adv_n = ppo_amd.gae_normalize(r, v, d, lv)
    from ppo_amd import _lib

    lib = _lib.load()
    ws = torch.empty(lib.ppo_gae_workspace_bytes(T, N), dtype=torch.uint8, device=dev)
    out, ret2 = torch.empty(T, N, device=dev), torch.empty(T, N, device=dev)
    rc = lib.ppo_gae_norm_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N, 0.99,
                              0.95, 1e-8, out.data_ptr(), ret2.data_ptr(), out.data_ptr(), None,
                              ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    assert torch.equal(out, adv_n) and torch.equal(ret2, ret)


def test_gae_out_may_not_alias_inputs_or_each_other(dev):
    """ops.gae / gae_normalize refuse caller outputs that overlap an input or
    each other (the passes read the value row after each segment while other
    workgroups store theirs); disjoint views of one buffer are accepted."""
    T, N = 64, 32
    r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.01, seed=9))
    adv, ret = ppo_amd.gae(r, v, d, lv)
    with pytest.raises(ValueError, match="overlaps"):
        ppo_amd.gae(r, v, d, lv, out=(v, torch.empty_like(r)))
    buf = torch.empty(3, T, N, device=dev)
    with pytest.raises(ValueError, match="overlaps"):
        ppo_amd.gae_normalize(r, v, d, lv, out=(buf[0], buf[0], buf[1]))
    a2, r2, n2 = ppo_amd.gae_normalize(r, v, d, lv, out=(buf[0], buf[1], buf[2]))
    torch.cuda.synchronize(dev)
    assert torch.equal(a2, adv) and torch.equal(r2, ret)


def test_discounted_returns_resident(dev):
    """values = None (REINFORCE returns) on the resident pass."""
    T, N = 4096, 512
    assert _route(T, N, False, has_values=False) == "resident"
    g = torch.Generator().manual_seed(9)
    r = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.01).to(torch.uint8)
    got = ppo_amd.discounted_returns(r.to(dev), gamma=0.97, dones=d.to(dev)).cpu().numpy()
    a_ref, _ = ref.gae_c(r.numpy(), np.zeros((T, N), np.float32), d.numpy(), None, 0.97, 1.0)
    assert_gae_close(got, a_ref)


def test_gae_resident_agrees_with_strip_walk_bitwise_mostly(dev, monkeypatch):
    """Config 2 on both routes: the same oracle bar, and the same bits in all
    but a few elements (they compose the carries in different orders)."""
    r, v, d, lv = (x.to(dev) for x in _inputs(2048, 4096, 0.01, seed=24))
    a1, _, n1 = ppo_amd.gae_normalize(r, v, d, lv)
    monkeypatch.setenv("PPO_AMD_GAE_RESIDENT", "0")
    a2, _, n2 = ppo_amd.gae_normalize(r, v, d, lv)
    same = float((a1 == a2).float().mean())
    print(f"  resident vs strip walk: {same:.6f} of advantages bit-identical", flush=True)
    assert same > 0.99
    torch.testing.assert_close(n1, n2, rtol=1e-5, atol=1e-6)


def test_gae_resident_non_finite_carry(dev):
    """An infinite value late in the horizon makes the carry entering the
    tiles to its left non-finite: elements whose recurrence reaches it through
    a done (0 * inf) are NaN, the others +-inf, exactly as the reference's
    float recurrence gives (the resident pass finishes carry-free segments
    before the look-back and must patch them)."""
    T, N = 2048, 1024
    assert _route(T, N, True) == "resident"
    r, v, d, lv = _inputs(T, N, 0.01, seed=10)
    v[1800, :8] = float("inf")
    v[1500, 8:12] = float("nan")
    print(f"gae resident non-finite T={T} N={N}", flush=True)
    adv, ret, _ = _gae_abi(dev, r.to(dev), v.to(dev), d.to(dev), lv.to(dev), 0.99, 0.95,
                           norm=True)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    got = adv.cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(a_ref))
    np.testing.assert_array_equal(np.isposinf(got), np.isposinf(a_ref))
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(a_ref))
    fin = np.isfinite(a_ref)
    assert np.isnan(a_ref).sum() > 1000  # the case is exercised
    assert_gae_close(got[fin], a_ref[fin])


# Rounds (no normaliser, rollouts longer than one resident grid): rounds of
# 256 tiles from the end of the horizon backwards, each handing the advantage
# at its left edge to the next; one to many env columns, a partial last round.
ROUND_SHAPES = [
    (1 << 20, 16, 0.001),   # config 3's shape: 16-env tiles, 2 rounds
    (1_000_003, 16, 0.001), # 16-env tiles, 2 rounds, the last tile ragged
    (600_000, 32, 0.002),   # 32-env tiles, 3 rounds, the last one partial
    (200_000, 128, 0.01),   # 2 columns x 128 tiles per round, 4 rounds
    (300_000, 64, 0.0),     # no dones: every carry crosses every tile and round
]


@pytest.mark.parametrize("T,N,p", ROUND_SHAPES)
def test_gae_resident_rounds_match_oracle(dev, T, N, p):
    assert _route(T, N, False) == "resident"
    exact, _, _ = _resident_case(dev, T, N, p, False, seed=T % 1000 + N)
    assert exact > 0.99


# Non-finite inputs on the resident pass without the normaliser.  Its
# look-back walks the composites from the nearest tile outwards and stops at
# the first whose factor product is zero (a done flag), skipping the tiles
# beyond; where a skipped tile holds an inf or NaN, the reference carries
# 0 x inf = NaN into every tile to its left, so the pass must find such tiles
# afterwards and write NaN there.  Non-finite values late in the horizon, in
# each round, and (one case) in the bootstrap value.
NONFINITE_SHAPES = [
    (16_384, 512, 0.002, False),  # one round, 32 tiles per column: walk window + full fold
    (1 << 20, 16, 0.001, False),  # config 3's shape: 16-env tiles, 2 rounds
    (600_000, 32, 0.002, True),   # 3 rounds, the last one partial; inf bootstrap value
    (300_000, 64, 0.0, False),    # no dones: carries cross every tile (inf, not NaN)
]


def _check_non_finite(dev, T, N, p, inf_last, seed):
    r, v, d, lv = _inputs(T, N, p, seed=seed)
    v[T - 100, 0] = float("inf")
    v[T - 5000, 1] = float("-inf")
    v[T // 2 + T // 7, 2] = float("nan")
    v[T // 3, 3] = float("inf")
    v[T // 3 + 7, 3] = float("-inf")   # meets the inf above: NaN from there on
    r[T // 5, N - 1] = float("inf")
    if inf_last:
        lv[N // 2] = float("inf")
    adv, ret, _ = _gae_abi(dev, r.to(dev), v.to(dev), d.to(dev), lv.to(dev), 0.99, 0.95)
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), lv.numpy(), 0.99, 0.95)
    got = adv.cpu().numpy()
    assert np.isnan(a_ref).sum() > 1000  # the case is exercised
    np.testing.assert_array_equal(np.isnan(got), np.isnan(a_ref))
    np.testing.assert_array_equal(np.isposinf(got), np.isposinf(a_ref))
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(a_ref))
    fin = np.isfinite(a_ref)
    assert_gae_close(got[fin], a_ref[fin])
    with np.errstate(invalid="ignore"):  # inf + -inf: NaN, as the kernel's fp32 sum gives
        ret_ref = got + v.numpy()
    np.testing.assert_array_equal(np.isnan(ret.cpu().numpy()), np.isnan(ret_ref))


@pytest.mark.parametrize("T,N,p,inf_last", NONFINITE_SHAPES)
def test_gae_resident_no_norm_non_finite(dev, T, N, p, inf_last):
    assert _route(T, N, False) == "resident"
    print(f"gae resident no-norm non-finite T={T} N={N} p={p} inf_last={inf_last}", flush=True)
    _check_non_finite(dev, T, N, p, inf_last, seed=T % 977 + N)


# The same on the other routes (resident pass off): carries composed over
# many tiles or spans without a done must keep an infinity as inf.
@pytest.mark.parametrize("T,N,p,route", [
    (1 << 17, 16, 0.0, "span"),
    (1 << 17, 16, 0.001, "span"),
    (100_000, 64, 0.0, "tiles"),
    (20_000, 100, 0.002, "tiles"),
    (16_384, 2048, 0.0, "strip"),
])
def test_gae_other_routes_non_finite(no_resident, dev, T, N, p, route):
    assert _route(T, N, False) == route
    print(f"gae {route} non-finite T={T} N={N} p={p}", flush=True)
    _check_non_finite(dev, T, N, p, True, seed=T % 991 + N)


def test_discounted_returns_resident_rounds(dev):
    """values = None (REINFORCE returns) in rounds."""
    T, N = 1 << 20, 16
    assert _route(T, N, False, has_values=False) == "resident"
    g = torch.Generator().manual_seed(19)
    r = torch.randn(T, N, generator=g)
    d = (torch.rand(T, N, generator=g) < 0.001).to(torch.uint8)
    got = ppo_amd.discounted_returns(r.to(dev), gamma=0.999, dones=d.to(dev)).cpu().numpy()
    a_ref, _ = ref.gae_c(r.numpy(), np.zeros((T, N), np.float32), d.numpy(), None, 0.999, 1.0)
    assert_gae_close(got, a_ref)


@pytest.mark.parametrize(
    "T,N,norm",
    [
        (2048, 4096, True),    # one round, 128-env tiles, with the normaliser
        (1024, 1024, True),    # one round, 64-env tiles, 4 steps per thread
        (200_000, 128, False), # rounds
    ],
)
def test_gae_resident_graph_replays_match_eager(dev, T, N, norm):
    """A captured resident-pass call replays with the nonce of its capture: the
    start barrier must reset the counters that the previous replay (or an eager
    call in between) completed.  Every replay, with new inputs copied in, and
    an eager call on the same workspace after it must equal a call on a fresh
    workspace bit for bit."""
    from ppo_amd import _lib

    lib = _lib.load()
    assert _route(T, N, norm) == "resident"
    print(f"gae resident graph replays T={T} N={N} norm={norm}", flush=True)
    g = torch.Generator(device=dev).manual_seed(T + N)

    def rollout():
        return (torch.randn(T, N, device=dev, generator=g), torch.randn(T, N, device=dev, generator=g),
                (torch.rand(T, N, device=dev, generator=g) < 0.01).to(torch.uint8),
                torch.randn(N, device=dev, generator=g))

    r, v, d, lv = rollout()
    ws = torch.full((lib.ppo_gae_workspace_bytes(T, N),), 0x5A, dtype=torch.uint8, device=dev)
    adv, ret, adv_n = (torch.empty(T, N, device=dev) for _ in range(3))

    def call():
        stream = torch.cuda.current_stream(dev).cuda_stream
        if norm:
            rc = lib.ppo_gae_norm_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N,
                                      0.99, 0.95, 1e-8, adv.data_ptr(), ret.data_ptr(),
                                      adv_n.data_ptr(), None, ws.data_ptr(), ws.numel(), stream)
        else:
            rc = lib.ppo_gae_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N,
                                 0.99, 0.95, adv.data_ptr(), ret.data_ptr(), ws.data_ptr(),
                                 ws.numel(), stream)
        assert rc == 0

    call()
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream(dev)):
        call()
    outs = (adv, ret, adv_n) if norm else (adv, ret)
    for rep in range(4):
        for dst, src in zip((r, v, d, lv), rollout()):
            dst.copy_(src)
        want = _gae_abi(dev, r, v, d, lv, 0.99, 0.95, norm=norm)
        graph.replay()
        torch.cuda.synchronize(dev)
        for got, w in zip(outs, want):
            assert torch.equal(got, w), f"replay {rep}"
        call()  # eager, same workspace, between replays
        torch.cuda.synchronize(dev)
        for got, w in zip(outs, want):
            assert torch.equal(got, w), f"eager after replay {rep}"


# ---------------------------------------------------------------------------
# Hyperparameter edges on every route, each against the oracle and against a
# closed form that does not use it: lambda = 0 gives the TD error
# ((r + (gamma * v') * mask) - v, ppo.py:180-184, in fp64, then fp32) and
# gamma = 0 gives r - v, both bit-exact; gamma = lambda = 1 with zero values,
# no dones and no bootstrap gives suffix sums of the rewards (fp64, to 1 ulp).
# ---------------------------------------------------------------------------
EDGE_ROUTES = [
    (2048, 1024, True),     # resident pass
    (2048, 1024, False),    # the same rollout off the resident pass
    (1 << 18, 16, True),    # resident pass in rounds
    (1 << 18, 16, False),   # span passes
    (300, 7, False),        # unaligned N: tile passes
]


@pytest.mark.parametrize("gamma,lam", [(0.99, 0.0), (0.0, 0.95), (1.0, 1.0), (0.9, 1.0)])
@pytest.mark.parametrize("T,N,resident", EDGE_ROUTES)
def test_gae_hyperparameter_edges(dev, monkeypatch, T, N, resident, gamma, lam):
    if not resident:
        monkeypatch.setenv("PPO_AMD_GAE_RESIDENT", "0")
    route = _route(T, N, False)
    assert (route == "resident") == resident
    suffix = gamma == 1.0 and lam == 1.0
    r, v, d, lv = _inputs(T, N, 0.0 if suffix else 0.01, seed=T + N + int(gamma * 10))
    if suffix:
        v.zero_()
        lv = None
    print(f"gae edges T={T} N={N} route={route} gamma={gamma} lam={lam}", flush=True)
    adv, _ = ppo_amd.gae(r.to(dev), v.to(dev), d.to(dev), None if lv is None else lv.to(dev),
                         gamma, lam)
    got = adv.cpu().numpy()
    a_ref, _ = ref.gae_c(r.numpy(), v.numpy(), d.numpy(), None if lv is None else lv.numpy(),
                         gamma, lam)
    assert_gae_close(got, a_ref)
    r64, v64 = r.numpy().astype(np.float64), v.numpy().astype(np.float64)
    mask = 1.0 - d.numpy().astype(np.float64)
    nv = np.concatenate([v64[1:], (np.zeros((1, N)) if lv is None else
                                   lv.numpy().astype(np.float64)[None, :])], axis=0)
    if lam == 0.0:
        want = ((r64 + (gamma * nv) * mask) - v64).astype(np.float32)
        np.testing.assert_array_equal(got, want)
    if gamma == 0.0:
        np.testing.assert_array_equal(got, (r64 - v64).astype(np.float32))
    if suffix:
        # (the carries between segments are composed in another order than
        # the serial sum, so <= 1 fp32 ulp as against the oracle)
        assert_gae_close(got, np.cumsum(r64[::-1], axis=0)[::-1])


@pytest.mark.parametrize("T,N", [(0, 8), (5, 0), (0, 0)])
def test_empty_rollouts(dev, T, N):
    """Empty rollouts give empty outputs without a launch; the fused
    normaliser's statistics of no elements are NaN, as torch's mean/std of an
    empty tensor."""
    r = torch.empty(T, N, device=dev)
    v = torch.empty(T, N, device=dev)
    d = torch.empty(T, N, dtype=torch.uint8, device=dev)
    lv = torch.empty(N, device=dev)
    adv, ret = ppo_amd.gae(r, v, d, lv)
    assert adv.shape == (T, N) and ret.shape == (T, N)
    adv, ret, adv_n, stats = ppo_amd.gae_normalize(r, v, d, lv, return_stats=True)
    assert adv_n.shape == (T, N)
    assert torch.isnan(stats).all()
    assert ppo_amd.normalize_advantages(adv).shape == (T, N)
    assert ppo_amd.discounted_returns(r, dones=d).shape == (T, N)


@pytest.mark.parametrize("T,N", [(2048, 4096), (2048, 64), (300, 4096), (1, 1), (5000, 3)])
def test_gae_normalise_in_place_matches_separate_outputs(dev, T, N):
    """keep_raw=False (adv_norm_out aliasing adv_out, the resident pass then
    storing no raw advantages) gives the normalised advantages and returns of
    the separate-output call bit for bit, on the resident route at the
    benchmark shape and on the other routes."""
    print(f"gae in place T={T} N={N}", flush=True)
    r, v, d, lv = (x.to(dev) for x in _inputs(T, N, 0.01, seed=31))
    adv, ret, adv_n, st = ppo_amd.gae_normalize(r, v, d, lv, return_stats=True)
    buf = torch.full((2, T, N), 7.0, device=dev)
    a2, r2, n2, st2 = ppo_amd.gae_normalize(r, v, d, lv, return_stats=True,
                                             out=(buf[0], buf[1]), keep_raw=False)
    torch.cuda.synchronize(dev)
    assert a2 is n2 and a2.data_ptr() == buf[0].data_ptr()
    assert torch.equal(n2, adv_n) and torch.equal(r2, ret)
    torch.testing.assert_close(st2, st, rtol=0, atol=0, equal_nan=True)
    if (T, N) == (2048, 4096):
        assert _route(T, N, True) == "resident"
    if T * N > 1:
        assert not torch.equal(n2, adv)
