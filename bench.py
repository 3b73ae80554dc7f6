"""PPO-update throughput on one MI355X.

A "step" is one pass of the PPO update hot path over one synthetic rollout of
T x N = 2048 x 4096 = 8,388,608 samples (the benchmark's GAE + normalise rollout):
  1. ppo_gae_norm_f32  — GAE with bootstrap + returns + advantage
                         normalisation (rl/deep/agents/ppo.py:123-127): the
                         advantages, returns and normalised advantages of
                         BASELINE config 2
  2. ppo_loss_cat_f32  — fused categorical PPO loss forward+backward over all
                         B = T*N samples, A = 18 actions, vf_clip = 0.2
                         (ppo.py:150-169; A = 18, value clipping 0.2)
Inputs are resident in HBM before the timed region.  `value` is samples/s
(B / step time).  `roofline` is for the dominant kernel (the fused loss:
172 algorithmic bytes per sample), timed with HIP events on the stream it is
launched on.  `cpu_baseline` times the CPU restatement of the same path
(oracle/, torch + numpy on the host cores) on a bounded sample.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--suite]

--suite additionally prints one line per benchmark configuration (2-5) kernel, for
the roofline table; --update-suite times the whole minibatch update loop;
the driver's contract line is always the last line.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "zero-to-hero_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
T_STEPS, N_ENVS, N_ACTIONS = 2048, 4096, 18
ROLLOUT_COPIES = 4  # rollouts the timed steps cycle through (4 x 75 MB > the 256 MB Infinity Cache)
GAE_BYTES = 21       # r 4 + V 4 + done 1 in; adv 4 + ret 4 + adv_n 4 out
GAE_INPLACE_BYTES = 17  # the same, normalised in place: ret 4 + adv_n 4 out
LOSS_CAT_BYTES = 172  # logits 72 + 6 x 4 per-row inputs in; dlogits 72 + dvalue 4 out
GAUSS_BYTES = 96     # mu 24 + actions 24 + 5 x 4 in; dmu 24 + dvalue 4 out
SCAN_BYTES = 17      # r, V, done in; adv, ret out
LOSS_CAT_A2_BYTES = 44  # A = 2: logits 8 + 6 x 4 in; dlogits 8 + dvalue 4 out


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--suite", action="store_true")
    ap.add_argument("--no-stream", action="store_true",
                    help="--suite without the back-to-back timing (us_stream), so that "
                         "profiler passes see only the isolated calls")
    ap.add_argument("--update-suite", action="store_true",
                    help="also time the whole minibatch update loop (VecPPO) vs the CPU oracle")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-clock budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gae-phases", metavar="LIB",
                    help="phase timestamps of the resident GAE pass (configs 2 and 3) from a "
                         "trace build of the library at LIB (make -C zero-to-hero_amd/csrc "
                         "EXTRA=-DPPO_GAE_RES_TRACE OBJDIR=_build_trace OUT=<LIB>); then exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (for rocprofv3 --pmc scaling)")
    return ap.parse_args()


def synthetic_rollout(torch, dev, T, N, A, seed=24):
    """The T x N rollout and the categorical loss inputs, generated on the GPU
    from a seeded generator."""
    g = torch.Generator(device=dev).manual_seed(seed)
    B = T * N
    x = {}
    x["rewards"] = torch.randn(T, N, device=dev, generator=g)
    x["values"] = torch.randn(T, N, device=dev, generator=g)
    x["dones"] = (torch.rand(T, N, device=dev, generator=g) < 0.01).to(torch.uint8)
    x["last_value"] = torch.randn(N, device=dev, generator=g)
    logits = torch.randn(B, A, device=dev, generator=g)
    old_logits = logits + 0.05 * torch.randn(B, A, device=dev, generator=g)
    # inverse-CDF sampling from softmax(old_logits), one column at a time
    probs = torch.softmax(old_logits, -1)
    u = torch.rand(B, device=dev, generator=g)
    acc = torch.zeros(B, device=dev)
    actions = torch.zeros(B, dtype=torch.int64, device=dev)
    for j in range(A - 1):
        acc += probs[:, j]
        actions += (u >= acc).to(torch.int64)
    x["old_log_probs"] = torch.log_softmax(old_logits, -1).gather(1, actions[:, None]).squeeze(1)
    del old_logits, probs, u, acc
    x["logits"] = logits
    x["actions"] = actions.to(torch.int32)
    x["new_values"] = x["values"].reshape(-1) + 0.1 * torch.randn(B, device=dev, generator=g)
    return x


ROLLOUT_KEYS = ("rewards", "values", "dones", "last_value")


class Step:
    """The two C-ABI calls of one update step, on torch's current stream,
    with preallocated outputs (nothing allocated inside the timed loop).
    The GAE call writes all three outputs BASELINE config 2 names
    (advantages, returns, normalised advantages: 21 bytes per sample with its
    inputs); `--suite` also times the in-place form the library's own update
    loop uses (config2_gae_norm_in_place).

    With copies > 1 the step keeps that many copies of the rollout (rewards,
    values, dones, last value: 75 MB each at T x N = 2048 x 4096) and next()
    moves to the following one, so that consecutive steps read different
    rollouts: together they exceed the 256 MB Infinity Cache, and a step's
    rollout comes from HBM, not from the cache lines the previous step left."""

    def __init__(self, torch, lib, x, dev, copies=1):
        import ctypes

        from ppo_amd import _lib

        self.torch, self.lib, self.x = torch, lib, x
        self.rollouts = [x] + [{k: x[k].clone() for k in ROLLOUT_KEYS}
                               for _ in range(copies - 1)]
        self.k = 0
        T, N = x["rewards"].shape
        B, A = x["logits"].shape
        self.T, self.N, self.B, self.A = T, N, B, A
        f32 = dict(dtype=torch.float32, device=dev)
        self.adv = torch.empty(T, N, **f32)
        self.ret = torch.empty(T, N, **f32)
        self.adv_n = torch.empty(T, N, **f32)
        self.stats = torch.empty(2, **f32)
        self.dlogits = torch.empty(B, A, **f32)
        self.dvalues = torch.empty(B, **f32)
        self.scalars = torch.empty(6, **f32)
        self.ws_gae = torch.zeros(lib.ppo_gae_workspace_bytes(T, N), dtype=torch.uint8, device=dev)
        self.ws_loss = torch.zeros(lib.ppo_loss_cat_workspace_bytes(B, A), dtype=torch.uint8,
                                   device=dev)
        self.params = _lib.LossParams(0.2, 0.2, 0.5, 0.01)
        self.params_ref = ctypes.byref(self.params)
        self.stream = torch.cuda.current_stream(dev).cuda_stream

    def next(self):
        self.k = (self.k + 1) % len(self.rollouts)

    def gae(self):
        x = self.rollouts[self.k]
        rc = self.lib.ppo_gae_norm_f32(
            x["rewards"].data_ptr(), x["values"].data_ptr(), x["dones"].data_ptr(),
            x["last_value"].data_ptr(), self.T, self.N, 0.99, 0.95, 1e-8,
            self.adv.data_ptr(), self.ret.data_ptr(), self.adv_n.data_ptr(),
            self.stats.data_ptr(), self.ws_gae.data_ptr(), self.ws_gae.numel(), self.stream)
        if rc:
            raise RuntimeError(f"ppo_gae_norm_f32 returned {rc}")

    def loss(self):
        x = self.x
        rc = self.lib.ppo_loss_cat_f32(
            x["logits"].data_ptr(), self.B, self.A, x["actions"].data_ptr(), 0,
            x["old_log_probs"].data_ptr(), self.adv_n.data_ptr(), self.ret.data_ptr(),
            x["new_values"].data_ptr(), self.rollouts[self.k]["values"].data_ptr(),
            self.params_ref,
            self.dlogits.data_ptr(), self.dvalues.data_ptr(), self.scalars.data_ptr(),
            self.ws_loss.data_ptr(), self.ws_loss.numel(), self.stream)
        if rc:
            raise RuntimeError(f"ppo_loss_cat_f32 returned {rc}")


def read_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    profiles/<name>.md (a line 'traffic_bytes_per_launch: <int>'), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}.md")
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def cpu_baseline(torch, x, budget_s):
    """The oracle's CPU path (GAE reverse loop vectorised over envs, torch
    normalisation, torch Categorical loss + autograd) on a bounded sample:
    the first `n_env` env columns of the same rollout over all T steps, and
    their T*n_env loss rows.  Repeats until `budget_s` seconds are used."""
    import numpy as np

    from oracle import ppo_oracle as ref

    T, N = x["rewards"].shape
    n_env = 128
    B = T * n_env
    cols = slice(0, n_env)
    r = x["rewards"][:, cols].cpu().numpy()
    v = x["values"][:, cols].cpu().numpy()
    d = x["dones"][:, cols].cpu().numpy()
    lv = x["last_value"][cols].cpu().numpy()
    rows = (torch.arange(T)[:, None] * N + torch.arange(n_env)[None, :]).reshape(-1)
    rows_d = rows.to(x["logits"].device)
    logits = x["logits"][rows_d].cpu()
    actions = x["actions"][rows_d].cpu()
    old_lp = x["old_log_probs"][rows_d].cpu()
    new_v = x["new_values"][rows_d].cpu()
    old_v = torch.from_numpy(np.ascontiguousarray(v)).reshape(-1)
    done_samples, t0 = 0, time.perf_counter()
    reps = 0
    while True:
        ref.cpu_update_step(r, v, d, lv, logits, actions, old_lp, new_v, old_v,
                            vf_clip=0.2)
        done_samples += B
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    # the reference's own scalar loop (ppo.py:177-190 semantics) at config 1's
    # shape: one T=128 episode per env column, N=8 columns, ~1 s of repeats
    g = np.random.default_rng(24)
    r1 = np.ones((128, 8))
    v1 = g.standard_normal((128, 8))
    d1 = g.random((128, 8)) < 1 / 200
    n1, t1 = 0, time.perf_counter()
    while time.perf_counter() - t1 < 1.0:
        for col in range(8):
            ref.advantages_python(r1[:, col].tolist(), d1[:, col].tolist(), v1[:, col].tolist(),
                                  0.99, 0.95)
        n1 += 128 * 8
    scalar_rate = n1 / (time.perf_counter() - t1)
    return {
        "value": done_samples / dt,
        "unit": "samples/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{reps} x (T={T} x {n_env} envs = {B} samples: GAE+norm+loss fwd/bwd, A=18)",
        "os_cpu_count": os.cpu_count(),
        "affinity_cores": len(os.sched_getaffinity(0)),
        "python_scalar_gae": {"value": round(scalar_rate), "unit": "elements/s", "cores": 1,
                              "sample": "oracle.advantages_python, T=128 x N=8 (config 1)"},
    }


def time_step_events(torch, step, reps):
    """Average durations (s) of step.gae() and step.loss() within `reps`
    back-to-back steps: HIP events before the GAE call, between the calls and
    after the loss call, on the current stream."""
    s = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
    for e in ev:
        e[0].record(s)
        step.gae()
        e[1].record(s)
        step.loss()
        e[2].record(s)
        step.next()
    torch.cuda.synchronize()
    g = sum(e[0].elapsed_time(e[1]) for e in ev) / reps / 1e3
    loss = sum(e[1].elapsed_time(e[2]) for e in ev) / reps / 1e3
    return g, loss


def time_events(torch, fn, reps, flush=None):
    """Average duration (s) of fn over `reps` launches, HIP events on the
    current stream (the stream the kernels are enqueued on).  `flush`, if
    given, runs before each launch, outside the events."""
    s = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        if flush is not None:
            flush()
        starts[i].record(s)
        fn()
        ends[i].record(s)
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in zip(starts, ends)]
    return sum(ms) / len(ms) / 1e3


def time_stream(torch, calls, passes):
    """Average duration (s) of one call when `calls` (one per buffer set) run
    back to back, `passes` times round, between two HIP events on the current
    stream.  The sets together are well over the 256 MB Infinity Cache, so
    each call's inputs come from HBM while the previous call's writes drain."""
    for fn in calls:
        fn()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(passes):
        for fn in calls:
            fn()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (passes * len(calls))


def suite(torch, lib, dev, stream_timing=True, cpu=True):
    """One line per benchmark configuration's kernel chain (2: GAE+normalise, 3: long-T
    GAE scan, 4: discrete loss, 5: Gaussian loss), each timed through the C
    ABI with preallocated outputs (HIP events on the launch stream), two ways:
    `us`, each timed call alone after a read of a 512 MiB buffer, so that its
    inputs come from HBM rather than the 256 MB Infinity Cache (configs 2, 4
    and 5 fit in it); and `us_stream`, calls back to back over several copies
    of the buffers (time_stream), without the idle time that event records
    around a single call leave on the device.  Unless `cpu` is False, each of
    configs 2-5 is also run once through the CPU restatement (oracle/) on the
    same inputs (`cpu_us`; config 3 through the C recurrence on one core, the
    others through numpy / torch on the host's threads).  `copy_us` /
    `copy_frac`: torch's device copy_ moving the same bytes, timed like `us`
    (the floor of a single timed call at that size); an `event_floor` line
    gives the event pair around no work."""
    import ctypes

    from ppo_amd import _lib

    g = torch.Generator(device=dev).manual_seed(24)
    stream = torch.cuda.current_stream(dev).cuda_stream
    f32 = dict(dtype=torch.float32, device=dev)
    params = _lib.LossParams(0.2, 0.2, 0.5, 0.01)
    out = []
    evict = torch.empty(128 * 1024 * 1024, **f32)
    evict_sum = torch.empty((), **f32)

    def flush():
        torch.sum(evict, dim=0, out=evict_sum)

    def ws(nbytes):
        return torch.empty(nbytes, dtype=torch.uint8, device=dev)

    cpu_us = {}

    def cpu_time(name, fn):
        if cpu:
            t0 = time.perf_counter()
            fn()
            cpu_us[name] = (time.perf_counter() - t0) * 1e6

    def measure(name, units, bpu, make, copies):
        """make(k) -> the call on buffer set k (set 0 also times `us`)."""
        calls = [make(k) for k in range(copies if stream_timing else 1)]
        calls[0]()
        t = time_events(torch, calls[0], 30, flush)
        out.append((name, units, bpu, t, time_stream(torch, calls, 8) if stream_timing else None))
        del calls

    # config 2 and 3: GAE over [T,N]
    for name, T, N, pd, gamma, norm, inplace, copies in (
            ("config2_gae_norm", 2048, 4096, 0.01, 0.99, True, False, 4),
            ("config2_gae_norm_in_place", 2048, 4096, 0.01, 0.99, True, True, 4),
            ("config3_long_scan", 1_048_576, 16, 0.001, 0.999, False, False, 3)):
        r = torch.randn(T, N, generator=g, **f32)
        v = torch.randn(T, N, generator=g, **f32)
        d = (torch.rand(T, N, device=dev, generator=g) < pd).to(torch.uint8)
        lv = torch.randn(N, generator=g, **f32)
        w = ws(lib.ppo_gae_workspace_bytes(T, N))

        def make(k, r=r, v=v, d=d, lv=lv, T=T, N=N, gamma=gamma, norm=norm, inplace=inplace,
                 w=w):
            if k:
                r, v, d = r.clone(), v.clone(), d.clone()
            adv, ret, advn = (torch.empty(T, N, **f32) for _ in range(3))
            if inplace:
                advn = adv
            if norm:
                return lambda: lib.ppo_gae_norm_f32(
                    r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N, gamma, 0.95,
                    1e-8, adv.data_ptr(), ret.data_ptr(), advn.data_ptr(), None, w.data_ptr(),
                    w.numel(), stream)
            return lambda: lib.ppo_gae_f32(
                r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N, gamma, 0.95,
                adv.data_ptr(), ret.data_ptr(), w.data_ptr(), w.numel(), stream)

        measure(name, T * N,
                (GAE_INPLACE_BYTES if inplace else GAE_BYTES) if norm else SCAN_BYTES, make, copies)
        if cpu and not inplace:
            from oracle import ppo_oracle as ref

            rn, vn, dn, ln = (t.cpu().numpy() for t in (r, v, d, lv))
            if norm:
                cpu_time(name, lambda: ref.normalize_reference(torch.from_numpy(
                    ref.gae_numpy(rn, vn, dn, ln, gamma, 0.95)[0]).reshape(-1)))
            else:
                ref.build_c()
                cpu_time(name, lambda: ref.gae_c(rn, vn, dn, ln, gamma, 0.95))
        del r, v, d, w, make
    # config 4: discrete loss
    x = synthetic_rollout(torch, dev, 256, 4096, 18, seed=25)
    B, A = x["logits"].shape
    sc = torch.empty(6, **f32)
    w = ws(lib.ppo_loss_cat_workspace_bytes(B, A))

    def make(k):
        y = x if k == 0 else {key: t.clone() for key, t in x.items()}
        dl, dv = torch.empty(B, A, **f32), torch.empty(B, **f32)
        return lambda: lib.ppo_loss_cat_f32(
            y["logits"].data_ptr(), B, A, y["actions"].data_ptr(), 0,
            y["old_log_probs"].data_ptr(), y["rewards"].data_ptr(), y["values"].data_ptr(),
            y["new_values"].data_ptr(), y["values"].data_ptr(), ctypes.byref(params),
            dl.data_ptr(), dv.data_ptr(), sc.data_ptr(), w.data_ptr(), w.numel(), stream)

    measure("config4_loss_cat", B, LOSS_CAT_BYTES, make, 4)
    if cpu:
        from oracle import ppo_oracle as ref

        xc = {key: t.cpu() for key, t in x.items()}
        cpu_time("config4_loss_cat", lambda: ref.loss_categorical_reference(
            xc["logits"], xc["actions"].long(), xc["old_log_probs"], xc["rewards"].reshape(-1),
            xc["values"].reshape(-1), xc["new_values"], xc["values"].reshape(-1), 0.2, 0.2,
            0.5, 0.01))
        del xc
    del x, w, make
    # config 5: Gaussian loss
    B, D = 2_097_152, 6
    mu = torch.randn(B, D, generator=g, **f32)
    ls = torch.rand(D, generator=g, **f32) - 1.0
    acts = mu + 0.05 * torch.randn(B, D, generator=g, **f32) + ls.exp() * torch.randn(
        B, D, generator=g, **f32)
    rows = [torch.randn(B, generator=g, **f32) for _ in range(5)]
    w = ws(lib.ppo_loss_gauss_workspace_bytes(B, D))

    def make(k):
        m, a_, rs = (mu, acts, rows) if k == 0 else (mu.clone(), acts.clone(),
                                                     [t.clone() for t in rows])
        dmu, dls, dv = torch.empty(B, D, **f32), torch.empty(D, **f32), torch.empty(B, **f32)
        return lambda: lib.ppo_loss_gauss_f32(
            m.data_ptr(), ls.data_ptr(), B, D, a_.data_ptr(), rs[0].data_ptr(),
            rs[1].data_ptr(), rs[2].data_ptr(), rs[3].data_ptr(), rs[4].data_ptr(),
            ctypes.byref(params), dmu.data_ptr(), dls.data_ptr(), dv.data_ptr(), sc.data_ptr(),
            w.data_ptr(), w.numel(), stream)

    measure("config5_loss_gauss", B, GAUSS_BYTES, make, 4)
    if cpu:
        from oracle import ppo_oracle as ref

        mc, lc, ac = mu.cpu(), ls.cpu(), acts.cpu()
        rc = [t.cpu() for t in rows]
        cpu_time("config5_loss_gauss", lambda: ref.loss_gaussian_reference(
            mc, lc, ac, rc[0], rc[1], rc[2], rc[3], rc[4], 0.2, 0.2, 0.5, 0.01))
        del mc, lc, ac, rc
    del mu, acts, rows, w, make
    # the north-star step with A = 2 (CartPole's action count): GAE+norm + loss
    x = synthetic_rollout(torch, dev, T_STEPS, N_ENVS, 2, seed=26)
    steps = [Step(torch, lib, x, dev)]
    if stream_timing:
        steps.append(Step(torch, lib, {key: t.clone() for key, t in x.items()}, dev))
    st = steps[0]
    st.gae()
    st.loss()
    out.append(("north_star_A2_loss", st.B, LOSS_CAT_A2_BYTES,
                time_events(torch, st.loss, 30, flush),
                time_stream(torch, [s_.loss for s_ in steps], 8) if stream_timing else None))
    out.append(("north_star_A2_step", st.B, GAE_BYTES + LOSS_CAT_A2_BYTES,
                time_events(torch, lambda: (st.gae(), st.loss()), 30, flush),
                time_stream(torch, [lambda s_=s_: (s_.gae(), s_.loss()) for s_ in steps], 8)
                if stream_timing else None))
    del steps, st, x
    # The floor of this timing at each byte count: torch's device copy_ moving
    # the same bytes (half read, half written), and an event pair around no
    # work, each after the same cache-evicting read.
    copy_us = {}
    for name, units, bpu, t, ts in out:
        n = units * bpu // 8
        src = torch.ones(n, **f32)
        dst = torch.empty_like(src)
        copy_us[name] = time_events(torch, lambda: dst.copy_(src), 30, flush)
        del src, dst
    floor = time_events(torch, lambda: None, 30, flush)
    print(json.dumps({"suite": "event_floor", "us": round(floor * 1e6, 2),
                      "what": "an event pair around no work, after the cache-evicting read"}),
          flush=True)
    for name, units, bpu, t, ts in out:
        gbs = units * bpu / t / 1e9
        line = {"suite": name, "units": units, "bytes_per_unit": bpu, "us": round(t * 1e6, 2),
                "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                "copy_us": round(copy_us[name] * 1e6, 2),
                "copy_frac": round(units * bpu / copy_us[name] / 1e9 / HBM_PEAK_GBS, 4)}
        if ts is not None:
            line["us_stream"] = round(ts * 1e6, 2)
            line["frac_stream"] = round(units * bpu / ts / 1e9 / HBM_PEAK_GBS, 4)
        if name in cpu_us:
            line["cpu_us"] = round(cpu_us[name], 1)
            line["cpu_threads"] = 1 if name == "config3_long_scan" else torch.get_num_threads()
        print(json.dumps(line), flush=True)


def update_suite(torch, dev, reps=10):
    """The whole update loop (ppo.py:113-171 generalised to [T,N]): GAE +
    normalisation + `epochs` x shuffled minibatches of MLP forward, fused loss,
    backward and optimizer step.  Configuration 1 (T=128, N=8, MLP 4-64-64
    tanh, A=2, 4 epochs x 4 minibatches of 256) and a larger T=2048, N=64 case
    (minibatches of 4096).  Times VecPPO with the fused MLP minibatch kernel +
    ClippedAdam replayed from graphs, the same eagerly, graph replay with
    torch's MLPs + the fused loss + gather, VecPPO with torch indexing +
    clip_grad_norm_ + Adam, and the CPU oracle (numpy GAE, torch CPU
    loss/backward/Adam)."""
    import copy

    import ppo_amd
    from oracle import ppo_oracle as ref
    from ppo_amd.agent import MLP, PPOConfig

    for name, T, N, mb in (("config1", 128, 8, 256), ("T2048_N64", 2048, 64, 4096)):
        g = torch.Generator().manual_seed(24)
        obs = (torch.rand(T, N, 4, generator=g) - 0.5) * 0.1
        torch.manual_seed(24)
        policy, value = MLP(4, 64, 2, "tanh"), MLP(4, 64, 1, "tanh")
        with torch.no_grad():
            logits = policy(obs)
            acts = torch.multinomial(torch.softmax(logits.reshape(-1, 2), -1), 1,
                                     generator=g).reshape(T, N)
            lps = torch.log_softmax(logits, -1).gather(2, acts[..., None]).squeeze(2)
            vals = value(obs).squeeze(2)
        rewards = torch.ones(T, N)
        dones = (torch.rand(T, N, generator=g) < 1 / 200).to(torch.uint8)
        buf = ppo_amd.RolloutBuffer(T, N, (4,), device=dev)
        for t in range(T):
            buf.add(obs[t].to(dev), acts[t].to(torch.int32).to(dev), rewards[t].to(dev),
                    dones[t].to(dev), vals[t].to(dev), lps[t].to(dev))
        buf.finish(None)
        out = {"update_suite": name, "T": T, "N": N, "minibatch": mb, "epochs": 4}
        for label, fused, graphs, fmlp in (("gpu_graphs_ms", True, True, True),
                                           ("gpu_fused_ms", True, False, True),
                                           ("gpu_graphs_torch_mlp_ms", True, True, False),
                                           ("gpu_torch_ms", False, False, False)):
            vec = ppo_amd.VecPPO(copy.deepcopy(policy).to(dev), copy.deepcopy(value).to(dev),
                                 PPOConfig(), batch_size=mb, fused_update=fused,
                                 generator=torch.Generator().manual_seed(7), graphs=graphs,
                                 fused_mlp=fmlp)
            vec.update(buf)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                vec.update(buf)
            torch.cuda.synchronize()
            out[label] = round((time.perf_counter() - t0) / reps * 1e3, 3)
        cpol, cval = copy.deepcopy(policy), copy.deepcopy(value)
        opt = torch.optim.Adam(list(cpol.parameters()) + list(cval.parameters()), lr=3e-4)
        cfg = ref.OracleConfig(batch_size=mb)
        gen = torch.Generator().manual_seed(7)
        t0 = time.perf_counter()
        creps = max(1, reps // 2)
        for _ in range(creps):
            adv, ret = ref.gae_numpy(rewards.numpy(), vals.numpy(), dones.numpy(), None,
                                     0.99, 0.95)
            adv_n = ref.normalize_reference(torch.from_numpy(adv).reshape(-1))
            ref.reference_epochs(cpol, cval, opt, obs.reshape(-1, 4), acts.reshape(-1),
                                 lps.reshape(-1), adv_n, torch.from_numpy(ret).reshape(-1), cfg,
                                 generator=gen)
        out["cpu_ms"] = round((time.perf_counter() - t0) / creps * 1e3, 3)
        out["cpu_threads"] = torch.get_num_threads()
        print(json.dumps(out), flush=True)
    dropin_agent_suite(torch, dev, reps)


def dropin_agent_suite(torch, dev, reps=10, T=500):
    """The drop-in PPOAgent as the reference's runner uses it, at the
    reference's defaults (TrainingConfig: hidden 128, ReLU, batch 128, 4
    epochs): `_update` over one T-step CartPole episode (ppo.py:113-171,
    steady state: every episode of a converged agent lasts 500 steps) and
    `select_action` (ppo.py:65-79), against oracle.ReferenceAgent (the same
    code path on the CPU, torch CPU ops) on the same rollout."""
    import numpy as np

    from oracle import ppo_oracle as ref
    from ppo_amd.agent import PPOAgent, TrainingConfig

    config = TrainingConfig()
    env = ref.CartPoleHost()
    gpu = PPOAgent(env, config, device=dev)
    cpu = ref.ReferenceAgent(hidden_size=config.hidden_size, batch_size=config.batch_size,
                             seed=config.seed)
    # one episode's rollout, collected by the CPU agent's own policy
    obs, _ = env.reset(seed=0)
    steps = []
    for t in range(T):
        a = cpu.select_action(obs)
        lp, v = cpu.pending
        nxt, r, term, trunc, _ = env.step(a)
        steps.append((obs, a, float(r), bool(term or trunc or t == T - 1), lp, v))
        obs = nxt if not (term or trunc) else env.reset(seed=t)[0]
    from ppo_amd.agent import RolloutStep, Transition
    gpu_rollout = [RolloutStep(Transition(o, a, r, o, d, False), lp, v)
                   for o, a, r, d, lp, v in steps]
    out = {"update_suite": "dropin_agent", "T": T, "hidden": config.hidden_size,
           "activation": "relu", "batch_size": config.batch_size, "epochs": 4,
           "fused_update": gpu.fused_update, "graphs": gpu.graphs}

    def gpu_update():
        gpu.rollout = gpu_rollout
        gpu._update()

    for _ in range(3):  # eager, capture, replay
        gpu_update()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        gpu_update()
    torch.cuda.synchronize()
    out["gpu_update_ms"] = round((time.perf_counter() - t0) / reps * 1e3, 3)
    t0 = time.perf_counter()
    creps = max(1, reps // 2)
    for _ in range(creps):
        cpu.rollout = list(steps)
        cpu.end_episode()
    out["cpu_update_ms"] = round((time.perf_counter() - t0) / creps * 1e3, 3)
    out["update_speedup"] = round(out["cpu_update_ms"] / out["gpu_update_ms"], 2)
    o = np.zeros(4, np.float32)
    for _ in range(20):
        gpu.select_action(o)
    n_act = 500
    t0 = time.perf_counter()
    for _ in range(n_act):
        gpu.select_action(o)
    out["gpu_select_action_us"] = round((time.perf_counter() - t0) / n_act * 1e6, 1)
    t0 = time.perf_counter()
    for _ in range(n_act):
        cpu.select_action(o)
    out["cpu_select_action_us"] = round((time.perf_counter() - t0) / n_act * 1e6, 1)
    out["cpu_threads"] = torch.get_num_threads()
    print(json.dumps(out), flush=True)


def gae_phases(torch, dev, lib_path, reps=4):
    """Phase timestamps of gae_resident_kernel from a trace build (each
    workgroup's thread 0 stores the wall clock, 100 MHz, at 6 marks per
    round into a device array the build exports): per config, per call
    after a cache-evicting read, the p50 and max over the workgroups of each
    mark, in us from the first workgroup's start, and the call's event
    interval."""
    import ctypes

    import numpy as np

    from ppo_amd import _lib

    lib = ctypes.CDLL(lib_path)
    for name, (res, argt) in _lib.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, argt
    lib.ppo_debug_res_trace.restype = ctypes.c_void_p
    hip = ctypes.CDLL("libamdhip64.so")
    row = 64  # trace words per workgroup (6 marks per round, up to 8 rounds)
    names = ["start", "phase1", "carry", "phase3", "stats", "end"]
    f32 = dict(dtype=torch.float32, device=dev)
    evict = torch.empty(128 * 1024 * 1024, **f32)
    es = torch.empty((), **f32)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for cfg, T, N, norm, gamma, p_done, rounds in (("config2", 2048, 4096, True, 0.99, 0.01, 1),
                                                   ("config3", 1 << 20, 16, False, 0.999, 0.001, 2)):
        g = torch.Generator(device=dev).manual_seed(24)
        r = torch.randn(T, N, generator=g, **f32)
        v = torch.randn(T, N, generator=g, **f32)
        d = (torch.rand(T, N, device=dev, generator=g) < p_done).to(torch.uint8)
        lv = torch.randn(N, generator=g, **f32)
        adv, ret, advn = (torch.empty(T, N, **f32) for _ in range(3))
        w = torch.empty(lib.ppo_gae_workspace_bytes(T, N), dtype=torch.uint8, device=dev)
        grid = None
        for rep in range(reps):
            # (marks a configuration does not write must not keep an earlier call's values)
            if hip.hipMemset(ctypes.c_void_p(lib.ppo_debug_res_trace()), 0,
                             ctypes.c_size_t(4096 * row * 8)):
                raise RuntimeError("hipMemset of the trace failed")
            torch.sum(evict, dim=0, out=es)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            if norm:
                rc = lib.ppo_gae_norm_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T,
                                          N, gamma, 0.95, 1e-8, adv.data_ptr(), ret.data_ptr(),
                                          advn.data_ptr(), None, w.data_ptr(), w.numel(), stream)
            else:
                rc = lib.ppo_gae_f32(r.data_ptr(), v.data_ptr(), d.data_ptr(), lv.data_ptr(), T, N,
                                     gamma, 0.95, adv.data_ptr(), ret.data_ptr(), w.data_ptr(),
                                     w.numel(), stream)
            e1.record()
            torch.cuda.synchronize()
            if rc:
                raise RuntimeError(f"GAE call returned {rc}")
            buf = np.zeros(4096 * row, dtype=np.uint64)
            if hip.hipMemcpy(buf.ctypes.data_as(ctypes.c_void_p),
                             ctypes.c_void_p(lib.ppo_debug_res_trace()),
                             ctypes.c_size_t(buf.nbytes), 2):
                raise RuntimeError("hipMemcpy of the trace failed")
            tr = buf.reshape(-1, row).astype(np.int64)
            if grid is None:
                grid = int((tr[:, 0] != 0).sum())
            tr = tr[:grid]
            rel = (tr - tr[:, 0].min()) / 100.0
            out = {"gae_phases": cfg, "T": T, "N": N, "rep": rep, "workgroups": grid,
                   "event_us": round(e0.elapsed_time(e1) * 1e3, 2)}
            for rd in range(rounds):
                for k, name in enumerate(names):
                    col = tr[:, k + 6 * rd]
                    if (rd > 0 and k == 0) or (col == 0).all():
                        continue
                    c = rel[:, k + 6 * rd]
                    out[f"r{rd}_{name}"] = [round(float(np.median(c)), 2), round(float(c.max()), 2)]
            print(json.dumps(out), flush=True)
        del r, v, d, adv, ret, advn, w


def copy_calibration(torch, dev, reps=3):
    """A plain device-to-device copy of exactly 1 GiB (torch copy_), run
    `reps` times so that a rocprofv3 --pmc pass over this command records what
    FETCH_SIZE / WRITE_SIZE report for 1 GiB read + 1 GiB written."""
    a = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import ppo_amd

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no CPU fallback)", file=sys.stderr)
        sys.exit(2)
    lib = ppo_amd.load_library()
    dev = torch.device("cuda:0")
    if args.gae_phases:
        gae_phases(torch, dev, args.gae_phases)
        return
    if args.suite:
        suite(torch, lib, dev, stream_timing=not args.no_stream, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
    if args.update_suite:
        update_suite(torch, dev)

    if args.copy_calibration:
        copy_calibration(torch, dev)
    x = synthetic_rollout(torch, dev, T_STEPS, N_ENVS, N_ACTIONS)
    step = Step(torch, lib, x, dev, copies=ROLLOUT_COPIES)
    B = step.B

    def one_step():
        step.gae()
        step.loss()
        step.next()

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3

    # per-call HIP-event timing on the launch stream, inside the step sequence
    # (each step reads the next of the rollout copies, so its rollout comes
    # from HBM)
    t_gae, t_loss = time_step_events(torch, step, max(args.steps, 20))
    achieved = LOSS_CAT_BYTES * B / t_loss / 1e9
    traffic = read_traffic("loss_cat_north_star")

    cpu = None if args.no_cpu else cpu_baseline(torch, x, args.cpu_seconds)

    line = {
        "metric": "PPO-update samples/sec (T×N=8M) + achieved HBM GB/s vs ~8 TB/s peak",
        "value": B / (ms_per_step / 1e3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (GAE recurrence in f64)",
        "data": "synthetic (seeded, BASELINE config-2 rollout + config-4 loss inputs)",
        "config": {
            "workload": "GAE+normalize (T=2048 x N=4096) + fused discrete PPO loss fwd/bwd "
                        "(B=8,388,608, A=18, vf_clip=0.2)",
            "T": T_STEPS, "N": N_ENVS, "A": N_ACTIONS, "samples_per_step": B,
        },
        "roofline": {
            "kernel": "ppo_loss_cat_f32 (loss_cat_wtile_kernel, finished in-kernel)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_sample": LOSS_CAT_BYTES,
            "avg_launch_us": round(t_loss * 1e6, 2),
        },
        "gae_norm": {
            "avg_call_us": round(t_gae * 1e6, 2),
            "bytes_per_sample": GAE_BYTES,
            "achieved_GBs": round(GAE_BYTES * B / t_gae / 1e9, 1),
            "frac": round(GAE_BYTES * B / t_gae / 1e9 / HBM_PEAK_GBS, 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
