"""Torch-facing ops over libppo_amd (HIP kernels for gfx950).

Each op validates its tensors on the host (device, dtype, shape, contiguity),
allocates outputs with torch, and enqueues the HIP kernels on torch's current
stream through the C ABI of include/ppo_amd.h.  Nothing here synchronises the
host, and nothing falls back to a CPU implementation: a missing library or a
non-CUDA tensor raises.

Reference functions replaced (mrhooray/zero-to-hero, rl/deep/agents/ppo.py):
  gae / gae_normalize     PPOAgent._advantages (:173-193), returns (:124),
                          normalisation (:126-127)
  normalize_advantages    ppo.py:126-127
  ppo_loss_discrete       PPOAgent._update_batch loss + backward (:150-169)
  ppo_loss_gaussian       the same loss for a Normal policy (no reference code)
  ppo_mlp_cat_grads       PPOAgent._update_batch forward + backward through the
                          actor/critic MLPs (:141-169, common.py:16-28)
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

__all__ = [
    "gae",
    "gae_normalize",
    "discounted_returns",
    "gather_rows",
    "normalize_advantages",
    "sample_categorical",
    "sample_gaussian",
    "ppo_loss_discrete",
    "ppo_loss_discrete_fused",
    "ppo_loss_gaussian",
    "ppo_loss_gaussian_fused",
    "ppo_mlp_cat_grads",
    "mlp_act_categorical",
    "mlp_forward_categorical",
    "mlp_fusable",
    "check_waits",
    "set_wait_limit",
    "WaitPoller",
    "LossStats",
]


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require(t: torch.Tensor, name: str, dtypes: tuple, device=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; ppo_amd runs on the GPU only (no CPU fallback)"
        )
    if device is not None and t.device != device:
        raise RuntimeError(f"{name} is on {t.device}, expected {device}")
    if t.dtype not in dtypes:
        names = ", ".join(str(d) for d in dtypes)
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {names}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _WorkspacePool:
    """One scratch buffer per (device, stream), grown on demand.

    libppo_amd needs caller-owned scratch (partial sums, tile carries).  Calls
    on one stream are ordered, so they can share a buffer; a different stream
    gets its own.
    """

    def __init__(self) -> None:
        self._bufs: dict = {}
        # while a graph is being captured: every buffer handed out is appended
        # here, so the graph keeps its scratch alive even if the pool later
        # replaces that buffer with a larger one
        self.capture_refs: Optional[list] = None

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device.index, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 0 if buf is None else 2 * buf.numel(), 4096)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        if self.capture_refs is not None:
            self.capture_refs.append(buf)
        return buf

    def drop(self, device: torch.device, stream: int) -> None:
        self._bufs.pop((device.index, stream), None)

    def zero(self, device: torch.device) -> None:
        """Zeroes every buffer of `device` (a zeroed workspace is valid for
        every entry point), on the current stream."""
        for (index, _), buf in self._bufs.items():
            if index == device.index:
                buf.zero_()


_WORKSPACES = _WorkspacePool()


def _call(name: str, device: torch.device, stream: int, *args) -> None:
    lib = _lib.load()
    code = getattr(lib, name)(*args)
    if code != _lib.PPO_OK:
        _WORKSPACES.drop(device, stream)
        _lib.check(name, code)


def check_waits(device: Optional[torch.device] = None) -> None:
    """Synchronises torch's current stream on `device` (default: the current
    device) and raises PPOLibraryError with code PPO_ERR_WAIT_TIMEOUT if a
    bounded in-kernel wait on that device gave up since the last check (on
    any stream).  The launches with such waits (the resident GAE pass, the
    Gaussian loss's in-kernel finish, the fused clip + Adam of
    ppo_mlp_cat_step) assume their whole grid runs at once; when another
    process or stream on the GPU prevents that, the affected outputs are NaN
    or the affected parameters unwritten, and this check reports it (and
    zeroes the pooled workspaces, which a late workgroup of the failed call
    may have left with stale arrival tags).  VecPPO.update and
    PPOAgent._update call it once per update."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(device):
        code = _lib.load().ppo_wait_status(_stream(device))
        if code == _lib.PPO_ERR_WAIT_TIMEOUT:
            # a late workgroup of the failed call may have left arrival tags
            # and counters in the workspaces: start them afresh
            _WORKSPACES.zero(device)
            torch.cuda.current_stream(device).synchronize()
        _lib.check("ppo_wait_status", code)


class WaitPoller:
    """Wait-status checks for a loop without a synchronisation per
    iteration (ppo_wait_status_async): check() enqueues this iteration's take
    of the device's status word into pinned host memory and reports the
    previous iteration's, waiting only for that earlier take (normally done:
    the GPU is then running this iteration's work).  A give-up is therefore
    reported by the check of the iteration after it, as a PPOLibraryError
    with code PPO_ERR_WAIT_TIMEOUT that covers every output since the last
    clean check; the pooled workspaces and the library's scratch are zeroed
    before it is raised.  flush() reports everything pending, synchronously."""

    def __init__(self) -> None:
        self._words: list = [None, None]
        self._events: list = [None, None]
        self._k = 0

    def _take(self, device: torch.device) -> None:
        k = self._k
        self._k ^= 1
        if self._words[k] is None:
            self._words[k] = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        stream = _stream(device)
        _lib.check("ppo_wait_status_async",
                   _lib.load().ppo_wait_status_async(self._words[k].data_ptr(), stream))
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        self._events[k] = ev

    def _pending(self, k: int) -> int:
        ev = self._events[k]
        if ev is None:
            return 0
        ev.synchronize()
        self._events[k] = None
        return int(self._words[k][0])

    def _fail(self, device: torch.device) -> None:
        for k in (0, 1):  # (a later take is covered by the same error)
            self._pending(k)
        _WORKSPACES.zero(device)
        _lib.check("ppo_wait_reset", _lib.load().ppo_wait_reset(_stream(device)))
        _lib.check("ppo_wait_status", _lib.PPO_ERR_WAIT_TIMEOUT)

    def check(self, device: torch.device) -> None:
        prev = self._k ^ 1
        with torch.cuda.device(device):
            self._take(device)
            if self._pending(prev):
                self._fail(device)

    def flush(self, device: torch.device) -> None:
        with torch.cuda.device(device):
            self._take(device)
            bad = self._pending(0) | self._pending(1)
            if bad:
                self._fail(device)


def set_wait_limit(polls: Optional[int]) -> None:
    """Poll limit of the bounded in-kernel waits launched from now on
    (process-wide): 0 makes every wait give up at once (tests of the failure
    path), None restores the default."""
    _lib.load().ppo_set_wait_limit(-1 if polls is None else int(polls))


def _as_2d(t: torch.Tensor) -> torch.Tensor:
    return t.unsqueeze(1) if t.dim() == 1 else t


def _done_bytes(dones: torch.Tensor) -> torch.Tensor:
    if dones.dtype == torch.bool:
        return dones.view(torch.uint8)
    return dones


# ---------------------------------------------------------------------------
# GAE and normalisation
# ---------------------------------------------------------------------------
def _gae_inputs(rewards, values, dones, last_value):
    _require(rewards, "rewards", (torch.float32,))
    device = rewards.device
    _require(values, "values", (torch.float32,), device)
    _require(dones, "dones", (torch.uint8, torch.bool), device)
    if rewards.dim() not in (1, 2):
        raise ValueError(f"rewards must be [T] or [T,N], got shape {tuple(rewards.shape)}")
    if values.shape != rewards.shape or dones.shape != rewards.shape:
        raise ValueError(
            "rewards, values and dones must share one shape, got "
            f"{tuple(rewards.shape)}, {tuple(values.shape)}, {tuple(dones.shape)}"
        )
    r2 = _as_2d(rewards)
    T, N = r2.shape
    if last_value is not None:
        _require(last_value, "last_value", (torch.float32,), device)
        if last_value.numel() != N:
            raise ValueError(f"last_value must hold N={N} values, got {last_value.numel()}")
    return device, T, N


def _span(t: torch.Tensor) -> tuple[int, int]:
    lo = t.data_ptr()
    return lo, lo + t.numel() * t.element_size()


def _outputs(out, count, like: torch.Tensor, inputs: tuple = ()) -> list:
    """Caller-provided output tensors (fp32, contiguous, the shape of `like`,
    on its device, overlapping neither each other nor `inputs`), or new ones.
    (The GAE passes read a row of values after each segment while other
    workgroups store theirs, so an output may not alias an input.)"""
    if out is None:
        return [torch.empty_like(like) for _ in range(count)]
    if len(out) != count:
        raise ValueError(f"out must hold {count} tensors, got {len(out)}")
    for k, t in enumerate(out):
        _require(t, f"out[{k}]", (torch.float32,), like.device)
        if t.shape != like.shape:
            raise ValueError(f"out[{k}] must have shape {tuple(like.shape)}, got {tuple(t.shape)}")
    spans = [_span(t) for t in out]
    others = spans + [_span(t) for t in inputs if t is not None and t.numel() > 0]
    for k, (lo, hi) in enumerate(spans):
        if hi > lo and any(j != k and lo < h and l < hi for j, (l, h) in enumerate(others)):
            raise ValueError(f"out[{k}] overlaps another output or an input")
    return list(out)


def gae(
    rewards: torch.Tensor,
    values: torch.Tensor,
    dones: torch.Tensor,
    last_value: Optional[torch.Tensor] = None,
    gamma: float = 0.99,
    lam: float = 0.95,
    out: Optional[tuple] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Advantages and returns of a [T,N] (or [T]) rollout on the GPU.

    Same recurrence as PPOAgent._advantages (ppo.py:173-193), per env, in fp64
    with the reference's operation order; `dones` is terminated-or-truncated
    (uint8 or bool); `last_value` [N] bootstraps past step T-1 (None = zeros,
    the reference's rule).  Returns (advantages, returns) fp32, same shape as
    rewards, with returns = advantages + values (ppo.py:124); written into
    `out` = (advantages, returns) when given.
    """
    device, T, N = _gae_inputs(rewards, values, dones, last_value)
    adv, ret = _outputs(out, 2, rewards, (rewards, values, dones, last_value))
    if T * N == 0:
        return adv, ret
    stream = _stream(device)
    nbytes = _lib.load().ppo_gae_workspace_bytes(T, N)
    ws = _WORKSPACES.get(device, stream, nbytes)
    _call(
        "ppo_gae_f32", device, stream,
        rewards.data_ptr(), values.data_ptr(), _done_bytes(dones).data_ptr(),
        _ptr(last_value), T, N, float(gamma), float(lam),
        adv.data_ptr(), ret.data_ptr(), ws.data_ptr(), ws.numel(), stream,
    )
    return adv, ret


def gae_normalize(
    rewards: torch.Tensor,
    values: torch.Tensor,
    dones: torch.Tensor,
    last_value: Optional[torch.Tensor] = None,
    gamma: float = 0.99,
    lam: float = 0.95,
    eps: float = 1e-8,
    return_stats: bool = False,
    out: Optional[tuple] = None,
    keep_raw: bool = True,
):
    """gae() plus the normalised advantages of ppo.py:126-127, fused: the
    advantage mean/std are accumulated inside the GAE pass.  Returns
    (advantages, returns, normalized_advantages[, stats]) where stats is a
    [2] fp32 device tensor {mean, std}; the first three are written into
    `out` when given.

    keep_raw=False drops the unnormalised advantages, as ppo.py:127 does by
    rebinding `advantages`: the normalised ones are written where the raw
    ones would be (the resident pass then skips one store per element), the
    returned tuple holds that tensor first and third, and `out` is
    (normalized_advantages, returns)."""
    device, T, N = _gae_inputs(rewards, values, dones, last_value)
    inputs = (rewards, values, dones, last_value)
    if keep_raw:
        adv, ret, adv_n = _outputs(out, 3, rewards, inputs)
    else:
        adv, ret = _outputs(out, 2, rewards, inputs)
        adv_n = adv
    stats = torch.empty(2, dtype=torch.float32, device=device)
    if T * N == 0:
        stats.fill_(float("nan"))  # torch's mean and std of no elements
    else:
        stream = _stream(device)
        nbytes = _lib.load().ppo_gae_workspace_bytes(T, N)
        ws = _WORKSPACES.get(device, stream, nbytes)
        _call(
            "ppo_gae_norm_f32", device, stream,
            rewards.data_ptr(), values.data_ptr(), _done_bytes(dones).data_ptr(),
            _ptr(last_value), T, N, float(gamma), float(lam), float(eps),
            adv.data_ptr(), ret.data_ptr(), adv_n.data_ptr(), stats.data_ptr(),
            ws.data_ptr(), ws.numel(), stream,
        )
    if return_stats:
        return adv, ret, adv_n, stats
    return adv, ret, adv_n


def normalize_advantages(
    advantages: torch.Tensor, eps: float = 1e-8, out: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """(adv - adv.mean()) / (adv.std() + eps) over all elements, unbiased std,
    and the identity for a single element (ppo.py:126-127)."""
    _require(advantages, "advantages", (torch.float32,))
    device = advantages.device
    if out is None:
        out = torch.empty_like(advantages)
    else:
        _require(out, "out", (torch.float32,), device)
        if out.shape != advantages.shape:
            raise ValueError("out must have the shape of advantages")
    n = advantages.numel()
    if n == 0:
        return out
    stream = _stream(device)
    nbytes = _lib.load().ppo_adv_norm_workspace_bytes(n)
    ws = _WORKSPACES.get(device, stream, nbytes)
    _call(
        "ppo_adv_norm_f32", device, stream,
        advantages.data_ptr(), n, float(eps), out.data_ptr(), None,
        ws.data_ptr(), ws.numel(), stream,
    )
    return out


def discounted_returns(
    rewards: torch.Tensor,
    dones: Optional[torch.Tensor] = None,
    gamma: float = 0.99,
    bootstrap: Optional[torch.Tensor] = None,
    center: bool = False,
) -> torch.Tensor:
    """REINFORCE returns, rl/deep/agents/reinforce.py:57-66, on the GPU.

    Per env, walking t backwards: value = reward + gamma * value, restarted
    after a done (the reference handles one episode, so it has no done inside
    the rollout), with `bootstrap` [N] (None = zeros, the reference's start
    value 0.0) entering after step T-1.  This is the GAE kernel with lambda = 1
    and all values zero, so the fp64 sums are bit-identical to the reference's
    Python floats.  With `center`, the mean over all returns is subtracted in
    fp32 (reinforce.py:66).
    """
    _require(rewards, "rewards", (torch.float32,))
    device = rewards.device
    if rewards.dim() not in (1, 2):
        raise ValueError(f"rewards must be [T] or [T,N], got shape {tuple(rewards.shape)}")
    if dones is None:
        dones = torch.zeros(rewards.shape, dtype=torch.uint8, device=device)
    _require(dones, "dones", (torch.uint8, torch.bool), device)
    if dones.shape != rewards.shape:
        raise ValueError("dones must have the shape of rewards")
    T, N = _as_2d(rewards).shape
    if bootstrap is not None:
        _require(bootstrap, "bootstrap", (torch.float32,), device)
        if bootstrap.numel() != N:
            raise ValueError(f"bootstrap must hold N={N} values, got {bootstrap.numel()}")
    out = torch.empty_like(rewards)
    if T * N == 0:
        return out
    stream = _stream(device)
    nbytes = _lib.load().ppo_gae_workspace_bytes(T, N)
    ws = _WORKSPACES.get(device, stream, nbytes)
    _call(
        "ppo_gae_f32", device, stream,
        rewards.data_ptr(), None, _done_bytes(dones).data_ptr(), _ptr(bootstrap), T, N,
        float(gamma), 1.0, out.data_ptr(), None, ws.data_ptr(), ws.numel(), stream,
    )
    if center:
        out = out - out.mean()
    return out


def gather_rows(index: torch.Tensor, *arrays: torch.Tensor) -> list[torch.Tensor]:
    """[a[index] for a in arrays] in one launch (the minibatch gather of
    ppo.py:132-139).  Every array is contiguous on one device with the same
    leading dimension n and 4-byte-multiple rows (fp32/int32/int64/...);
    `index` is int64 [B] with values in [0, n) (others give zero rows)."""
    _require(index, "index", (torch.int64,))
    device = index.device
    if index.dim() != 1:
        raise ValueError(f"index must be 1-D, got shape {tuple(index.shape)}")
    if not 1 <= len(arrays) <= _lib.GATHER_MAX_ARRAYS:
        raise ValueError(f"between 1 and {_lib.GATHER_MAX_ARRAYS} arrays, got {len(arrays)}")
    n = arrays[0].shape[0]
    outs, rb = [], []
    for k, a in enumerate(arrays):
        if not isinstance(a, torch.Tensor) or a.device != device:
            raise RuntimeError(f"array {k} must be a tensor on {device}")
        if not a.is_contiguous():
            raise ValueError(f"array {k} must be contiguous")
        if a.dim() < 1 or a.shape[0] != n:
            raise ValueError(f"array {k} must have leading dimension {n}")
        row = a.element_size() * (a[0].numel() if a.dim() > 1 else 1)
        if row % 4:
            raise ValueError(f"array {k}: rows of {row} bytes are not a multiple of 4")
        rb.append(row)
        outs.append(torch.empty((index.numel(),) + tuple(a.shape[1:]), dtype=a.dtype,
                                device=device))
    B = index.numel()
    if B == 0:
        return outs
    na = len(arrays)
    src = (ctypes.c_void_p * na)(*[a.data_ptr() for a in arrays])
    dst = (ctypes.c_void_p * na)(*[o.data_ptr() for o in outs])
    rbs = (ctypes.c_int32 * na)(*rb)
    stream = _stream(device)
    _call("ppo_gather_rows", device, stream, index.data_ptr(), B, n, na, src, rbs, dst, stream)
    return outs


def copy_pinned_to_device(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """dst <- src for a pinned host tensor `src`, as one kernel launch on the
    current stream that reads the pinned memory over the bus
    (ppo_copy_from_pinned).  Asynchronous: the host must not overwrite `src`
    until the stream has passed this launch (record an event).  A small
    host-to-device copy through the runtime can instead wait for the stream's
    earlier work and stall the host."""
    if not isinstance(src, torch.Tensor) or src.device.type != "cpu" or not src.is_pinned():
        raise ValueError("src must be a pinned host tensor")
    if not src.is_contiguous() or not dst.is_contiguous():
        raise ValueError("src and dst must be contiguous")
    if dst.device.type != "cuda" or dst.dtype != src.dtype or dst.numel() != src.numel():
        raise ValueError("dst must be a CUDA tensor of src's dtype and size")
    nbytes = src.numel() * src.element_size()
    device = dst.device
    stream = _stream(device)
    _call("ppo_copy_from_pinned", device, stream, dst.data_ptr(), src.data_ptr(), nbytes, stream)
    return dst


# ---------------------------------------------------------------------------
# Batched action selection
# ---------------------------------------------------------------------------
def _out(t, name, shape, dtype, device):
    if t is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _require(t, name, (dtype,), device)
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    return t


def sample_categorical(
    logits: torch.Tensor,
    uniforms: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
    values: Optional[torch.Tensor] = None,
    actions_out: Optional[torch.Tensor] = None,
    log_probs_out: Optional[torch.Tensor] = None,
    values_out: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Categorical(logits=logits).sample() and .log_prob() for N rows in one
    launch (PPOAgent.select_action, ppo.py:65-79, batched over envs).

    The draw is the inverse CDF of softmax(logits[n]) at uniforms[n] (drawn
    with torch.rand on the device from `generator` when not given), so the
    sample is a deterministic function of (logits, uniforms).  Returns
    (actions int32 [N], log_probs [N]); the *_out tensors, if given, are
    written in place (e.g. row t of a [T,N] rollout buffer), and `values`
    is copied to `values_out` in the same launch.
    """
    _require(logits, "logits", (torch.float32,))
    device = logits.device
    if logits.dim() != 2 or logits.shape[1] == 0:
        raise ValueError(f"logits must be [N,A] with A > 0, got {tuple(logits.shape)}")
    N, A = logits.shape
    if uniforms is None:
        uniforms = torch.rand(N, device=device, generator=generator)
    _require(uniforms, "uniforms", (torch.float32,), device)
    if uniforms.shape != (N,):
        raise ValueError(f"uniforms must be [N]=[{N}], got {tuple(uniforms.shape)}")
    actions_out = _out(actions_out, "actions_out", (N,), torch.int32, device)
    log_probs_out = _out(log_probs_out, "log_probs_out", (N,), torch.float32, device)
    if (values is None) != (values_out is None):
        raise ValueError("values and values_out go together")
    if values is not None:
        _require(values, "values", (torch.float32,), device)
        values_out = _out(values_out, "values_out", (N,), torch.float32, device)
        if values.numel() != N:
            raise ValueError(f"values must have N={N} elements, got {values.numel()}")
    stream = _stream(device)
    _call("ppo_sample_cat_f32", device, stream, logits.data_ptr(), N, A, uniforms.data_ptr(),
          actions_out.data_ptr(), log_probs_out.data_ptr(), _ptr(values), _ptr(values_out),
          stream)
    return actions_out, log_probs_out


def sample_gaussian(
    mu: torch.Tensor,
    log_std: torch.Tensor,
    normals: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
    values: Optional[torch.Tensor] = None,
    actions_out: Optional[torch.Tensor] = None,
    log_probs_out: Optional[torch.Tensor] = None,
    values_out: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Normal(mu, exp(log_std)).sample() and .log_prob(a).sum(-1) for N rows
    in one launch: actions = mu + exp(log_std) * normals (normals drawn with
    torch.randn from `generator` when not given).  Returns (actions [N,D],
    log_probs [N]); *_out tensors are written in place when given."""
    _require(mu, "mu", (torch.float32,))
    device = mu.device
    if mu.dim() != 2 or mu.shape[1] == 0:
        raise ValueError(f"mu must be [N,D] with D > 0, got {tuple(mu.shape)}")
    N, D = mu.shape
    _require(log_std, "log_std", (torch.float32,), device)
    if log_std.numel() != D:
        raise ValueError(f"log_std must have D={D} elements, got {log_std.numel()}")
    if normals is None:
        normals = torch.randn(N, D, device=device, generator=generator)
    _require(normals, "normals", (torch.float32,), device)
    if normals.shape != (N, D):
        raise ValueError(f"normals must be [N,D]=[{N},{D}], got {tuple(normals.shape)}")
    actions_out = _out(actions_out, "actions_out", (N, D), torch.float32, device)
    log_probs_out = _out(log_probs_out, "log_probs_out", (N,), torch.float32, device)
    if (values is None) != (values_out is None):
        raise ValueError("values and values_out go together")
    if values is not None:
        _require(values, "values", (torch.float32,), device)
        values_out = _out(values_out, "values_out", (N,), torch.float32, device)
        if values.numel() != N:
            raise ValueError(f"values must have N={N} elements, got {values.numel()}")
    stream = _stream(device)
    _call("ppo_sample_gauss_f32", device, stream, mu.data_ptr(), log_std.contiguous().data_ptr(),
          N, D, normals.data_ptr(), actions_out.data_ptr(), log_probs_out.data_ptr(),
          _ptr(values), _ptr(values_out), stream)
    return actions_out, log_probs_out


# ---------------------------------------------------------------------------
# Fused loss
# ---------------------------------------------------------------------------
class LossStats(dict):
    """Loss scalars as 0-d fp32 device tensors: loss, policy, value, entropy,
    approx_kl, clipfrac (views of one [6] tensor; no host sync)."""


def _stats_dict(scalars: torch.Tensor) -> LossStats:
    s = scalars.detach()
    return LossStats({name: s[i] for i, name in enumerate(_lib.SCALAR_NAMES)})


def _params(clip_ratio, vf_clip, value_coef, entropy_coef) -> _lib.LossParams:
    if not clip_ratio >= 0.0:
        raise ValueError(f"clip_ratio must be >= 0, got {clip_ratio}")
    vc = 0.0 if vf_clip is None else float(vf_clip)
    if vf_clip is not None and not vc > 0.0:
        raise ValueError(f"vf_clip must be > 0 or None, got {vf_clip}")
    return _lib.LossParams(float(clip_ratio), vc, float(value_coef), float(entropy_coef))


def _row_inputs(device, B, old_log_probs, advantages, returns, values, old_values, vf_clip):
    for t, name in (
        (old_log_probs, "old_log_probs"),
        (advantages, "advantages"),
        (returns, "returns"),
        (values, "values"),
    ):
        _require(t, name, (torch.float32,), device)
        if t.numel() != B or t.dim() != 1:
            raise ValueError(f"{name} must be [B]=[{B}], got {tuple(t.shape)}")
    if vf_clip is not None:
        if old_values is None:
            raise ValueError("old_values is required when vf_clip is set")
    if old_values is not None:
        _require(old_values, "old_values", (torch.float32,), device)
        if old_values.numel() != B or old_values.dim() != 1:
            raise ValueError(f"old_values must be [B]=[{B}], got {tuple(old_values.shape)}")


def ppo_loss_discrete_fused(
    logits: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
    validate_args: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One launch of the fused categorical PPO loss forward+backward.

    Returns (scalars[6], dlogits[B,A], dvalues[B]) with scalars ordered as
    LossStats; the gradients are d loss / d logits and d loss / d values.
    With validate_args, out-of-range actions raise ValueError as
    torch.distributions.Categorical's support check does (this syncs);
    without it, such a row's log-prob is NaN.
    """
    _require(logits, "logits", (torch.float32,))
    device = logits.device
    if logits.dim() != 2:
        raise ValueError(f"logits must be [B,A], got {tuple(logits.shape)}")
    B, A = logits.shape
    _require(actions, "actions", (torch.int32, torch.int64), device)
    if actions.numel() != B or actions.dim() != 1:
        raise ValueError(f"actions must be [B]=[{B}], got {tuple(actions.shape)}")
    _row_inputs(device, B, old_log_probs, advantages, returns, values, old_values, vf_clip)
    if B == 0 or A == 0:
        raise ValueError("logits must have B > 0 rows and A > 0 actions")
    if validate_args:
        bad = ((actions < 0) | (actions >= A)).any()
        if bool(bad):
            raise ValueError(
                "The value argument must be within the support of the categorical "
                f"distribution (actions in [0, {A}))"
            )
    params = _params(clip_ratio, vf_clip, value_coef, entropy_coef)
    dlogits = torch.empty_like(logits)
    dvalues = torch.empty_like(values)
    scalars = torch.empty(_lib.PPO_NUM_SCALARS, dtype=torch.float32, device=device)
    stream = _stream(device)
    nbytes = _lib.load().ppo_loss_cat_workspace_bytes(B, A)
    ws = _WORKSPACES.get(device, stream, nbytes)
    _call(
        "ppo_loss_cat_f32", device, stream,
        logits.data_ptr(), B, A, actions.data_ptr(), int(actions.dtype == torch.int64),
        old_log_probs.data_ptr(), advantages.data_ptr(), returns.data_ptr(),
        values.data_ptr(), _ptr(old_values), ctypes.byref(params),
        dlogits.data_ptr(), dvalues.data_ptr(), scalars.data_ptr(),
        ws.data_ptr(), ws.numel(), stream,
    )
    return scalars, dlogits, dvalues


class _DiscreteLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, values, actions, old_log_probs, advantages, returns,
                old_values, clip_ratio, vf_clip, value_coef, entropy_coef, validate_args):
        scalars, dlogits, dvalues = ppo_loss_discrete_fused(
            logits.detach(), actions, old_log_probs, advantages, returns, values.detach(),
            old_values, clip_ratio, vf_clip, value_coef, entropy_coef, validate_args,
        )
        ctx.save_for_backward(dlogits, dvalues)
        return scalars

    @staticmethod
    def backward(ctx, grad_scalars):
        dlogits, dvalues = ctx.saved_tensors
        g = grad_scalars[0]
        return (dlogits * g, dvalues * g) + (None,) * 10


def ppo_loss_discrete(
    logits: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
    validate_args: bool = False,
) -> tuple[torch.Tensor, LossStats]:
    """Differentiable PPO loss of a categorical policy (ppo.py:150-167).

    Returns (loss, stats): `loss` is a 0-d tensor whose backward delivers the
    fused kernel's d loss / d logits and d loss / d values (scaled by the
    incoming gradient); `stats` holds the component scalars, which are
    reported values, not differentiable outputs.
    """
    scalars = _DiscreteLoss.apply(
        logits, values, actions, old_log_probs, advantages, returns, old_values,
        clip_ratio, vf_clip, value_coef, entropy_coef, validate_args,
    )
    return scalars[0], _stats_dict(scalars)


def ppo_loss_gaussian_fused(
    mu: torch.Tensor,
    log_std: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """One launch of the fused Gaussian PPO loss forward+backward.

    Policy Normal(mu, exp(log_std)), log_std [D] state-independent, log-prob
    and entropy summed over D.  Returns (scalars[6], dmu[B,D], dlog_std[D],
    dvalues[B]).
    """
    _require(mu, "mu", (torch.float32,))
    device = mu.device
    if mu.dim() != 2:
        raise ValueError(f"mu must be [B,D], got {tuple(mu.shape)}")
    B, D = mu.shape
    if B == 0 or D == 0:
        raise ValueError("mu must have B > 0 rows and D > 0 dims")
    if D > 24:
        raise ValueError(f"action dim D={D} exceeds the kernel's limit of 24")
    _require(log_std, "log_std", (torch.float32,), device)
    if log_std.numel() != D or log_std.dim() != 1:
        raise ValueError(f"log_std must be [D]=[{D}], got {tuple(log_std.shape)}")
    _require(actions, "actions", (torch.float32,), device)
    if actions.shape != mu.shape:
        raise ValueError(f"actions must be [B,D]={tuple(mu.shape)}, got {tuple(actions.shape)}")
    _row_inputs(device, B, old_log_probs, advantages, returns, values, old_values, vf_clip)
    params = _params(clip_ratio, vf_clip, value_coef, entropy_coef)
    dmu = torch.empty_like(mu)
    dlog_std = torch.empty_like(log_std)
    dvalues = torch.empty_like(values)
    scalars = torch.empty(_lib.PPO_NUM_SCALARS, dtype=torch.float32, device=device)
    stream = _stream(device)
    nbytes = _lib.load().ppo_loss_gauss_workspace_bytes(B, D)
    ws = _WORKSPACES.get(device, stream, nbytes)
    _call(
        "ppo_loss_gauss_f32", device, stream,
        mu.data_ptr(), log_std.data_ptr(), B, D, actions.data_ptr(),
        old_log_probs.data_ptr(), advantages.data_ptr(), returns.data_ptr(),
        values.data_ptr(), _ptr(old_values), ctypes.byref(params),
        dmu.data_ptr(), dlog_std.data_ptr(), dvalues.data_ptr(), scalars.data_ptr(),
        ws.data_ptr(), ws.numel(), stream,
    )
    return scalars, dmu, dlog_std, dvalues


class _GaussianLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, mu, log_std, values, actions, old_log_probs, advantages, returns,
                old_values, clip_ratio, vf_clip, value_coef, entropy_coef):
        scalars, dmu, dlog_std, dvalues = ppo_loss_gaussian_fused(
            mu.detach(), log_std.detach(), actions, old_log_probs, advantages, returns,
            values.detach(), old_values, clip_ratio, vf_clip, value_coef, entropy_coef,
        )
        ctx.save_for_backward(dmu, dlog_std, dvalues)
        return scalars

    @staticmethod
    def backward(ctx, grad_scalars):
        dmu, dlog_std, dvalues = ctx.saved_tensors
        g = grad_scalars[0]
        return (dmu * g, dlog_std * g, dvalues * g) + (None,) * 9


def ppo_loss_gaussian(
    mu: torch.Tensor,
    log_std: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    values: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
) -> tuple[torch.Tensor, LossStats]:
    """Differentiable PPO loss of a Normal(mu, exp(log_std)) policy; gradients
    reach mu, log_std and values.  See ppo_loss_discrete for the contract."""
    scalars = _GaussianLoss.apply(
        mu, log_std, values, actions, old_log_probs, advantages, returns, old_values,
        clip_ratio, vf_clip, value_coef, entropy_coef,
    )
    return scalars[0], _stats_dict(scalars)


# ---------------------------------------------------------------------------
# Fused minibatch gradient through the actor and critic MLPs
# ---------------------------------------------------------------------------
MLP_HIDDEN_SIZES = (16, 32, 64, 128)
MLP_MAX_IN = 64
MLP_MAX_ACTIONS = 32


def mlp_structure(net: torch.nn.Module) -> Optional[tuple[list, str]]:
    """The three nn.Linear layers and the activation ("relu" / "tanh") of a
    network shaped like rl/deep/agents/common.py:16-28's MLP (an `.net`
    nn.Sequential, or the Sequential itself, of Linear-act-Linear-act-Linear
    with one activation), or None for any other network."""
    seq = getattr(net, "net", net)
    if not isinstance(seq, torch.nn.Sequential) or len(seq) != 5:
        return None
    lin = [seq[0], seq[2], seq[4]]
    if not all(type(m) is torch.nn.Linear and m.bias is not None for m in lin):
        return None
    kinds = {type(seq[1]), type(seq[3])}
    if kinds == {torch.nn.ReLU}:
        act = "relu"
    elif kinds == {torch.nn.Tanh}:
        act = "tanh"
    else:
        return None
    return lin, act


def mlp_fusable(policy: torch.nn.Module, value: torch.nn.Module) -> bool:
    """True when ppo_mlp_cat_grads supports this actor/critic pair: both
    MLP-shaped with the same input size, hidden size (16/32/64/128) and
    activation, the critic with one output, <= 64 inputs, <= 32 actions, fp32
    contiguous parameters on one GPU."""
    sp, sv = mlp_structure(policy), mlp_structure(value)
    if sp is None or sv is None or sp[1] != sv[1]:
        return False
    lp, lv = sp[0], sv[0]
    D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
    if lv[0].in_features != D or lv[0].out_features != H or lv[2].out_features != 1:
        return False
    if lp[1].in_features != H or lp[1].out_features != H or lv[1].out_features != H:
        return False
    if H not in MLP_HIDDEN_SIZES or D > MLP_MAX_IN or A > MLP_MAX_ACTIONS:
        return False
    params = [p for m in lp + lv for p in (m.weight, m.bias)]
    dev = params[0].device
    return all(p.device == dev and p.device.type == "cuda" and p.dtype == torch.float32
               and p.is_contiguous() for p in params)


def _mlp_struct(layers: list) -> _lib.Mlp3:
    s = _lib.Mlp3()
    for i, m in enumerate(layers):
        for p in (m.weight, m.bias):
            if p.grad is None:
                p.grad = torch.zeros_like(p)
            elif p.grad.shape != p.shape or p.grad.dtype != p.dtype or not p.grad.is_contiguous():
                raise ValueError("parameter gradients must be contiguous fp32 of the parameter's shape")
        s.weight[i] = m.weight.data_ptr()
        s.bias[i] = m.bias.data_ptr()
        s.weight_grad[i] = m.weight.grad.data_ptr()
        s.bias_grad[i] = m.bias.grad.data_ptr()
    return s


def _mlp_minibatch_args(policy, value, observations, actions, old_log_probs, advantages,
                        returns, old_values, index, clip_ratio, vf_clip, value_coef,
                        entropy_coef, scalars_out):
    """Validated arguments of the fused minibatch entry points (the part of
    their C signatures they share), the device, stream and workspace."""
    if not mlp_fusable(policy, value):
        raise ValueError("policy/value are not MLPs the fused kernel supports (see mlp_fusable)")
    lp, act = mlp_structure(policy)
    lv, _ = mlp_structure(value)
    D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
    device = lp[0].weight.device
    _require(observations, "observations", (torch.float32,), device)
    if observations.dim() != 2 or observations.shape[1] != D:
        raise ValueError(f"observations must be [n,{D}], got {tuple(observations.shape)}")
    n = observations.shape[0]
    _require(actions, "actions", (torch.int32, torch.int64), device)
    if actions.shape != (n,):
        raise ValueError(f"actions must be [n]=[{n}], got {tuple(actions.shape)}")
    for t, name in ((old_log_probs, "old_log_probs"), (advantages, "advantages"),
                    (returns, "returns")):
        _require(t, name, (torch.float32,), device)
        if t.shape != (n,):
            raise ValueError(f"{name} must be [n]=[{n}], got {tuple(t.shape)}")
    params = _params(clip_ratio, vf_clip, value_coef, entropy_coef)
    if vf_clip is not None:
        if old_values is None:
            raise ValueError("vf_clip needs old_values")
        _require(old_values, "old_values", (torch.float32,), device)
        if old_values.shape != (n,):
            raise ValueError(f"old_values must be [n]=[{n}], got {tuple(old_values.shape)}")
    if index is not None:
        _require(index, "index", (torch.int64,), device)
        if index.dim() != 1:
            raise ValueError(f"index must be 1-D, got {tuple(index.shape)}")
        B = index.numel()
    else:
        B = n
    if B == 0:
        raise ValueError("the minibatch is empty")
    scalars = _out(scalars_out, "scalars_out", (_lib.PPO_NUM_SCALARS,), torch.float32, device)
    actor, critic = _mlp_struct(lp), _mlp_struct(lv)
    stream = _stream(device)
    nbytes = _lib.load().ppo_mlp_cat_grad_workspace_bytes(B, D, H, A)
    ws = _WORKSPACES.get(device, stream, nbytes)
    head = (ctypes.byref(actor), ctypes.byref(critic), D, H, A,
            _lib.PPO_ACT_TANH if act == "tanh" else _lib.PPO_ACT_RELU,
            observations.data_ptr(), n, _ptr(index), B, actions.data_ptr(),
            1 if actions.dtype == torch.int64 else 0, old_log_probs.data_ptr(),
            advantages.data_ptr(), returns.data_ptr(),
            _ptr(old_values) if vf_clip is not None else None, ctypes.byref(params))
    # the ctypes structs must outlive the call
    return device, stream, ws, scalars, head, (actor, critic, params)


def ppo_mlp_cat_grads(
    policy: torch.nn.Module,
    value: torch.nn.Module,
    observations: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    index: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
    scalars_out: Optional[torch.Tensor] = None,
) -> LossStats:
    """Forward and backward of PPOAgent._update_batch (ppo.py:141-169) for one
    minibatch in two launches: the rows `index` (int64 [B]; None: all n rows)
    of the rollout arrays (observations [n,D], actions [n] int32/int64,
    old_log_probs / advantages / returns / old_values [n]) go through both
    MLPs, the categorical PPO loss and its backward, and every parameter's
    `.grad` is overwritten with d loss / d parameter (allocated if None).
    Returns the loss scalars (0-d device tensors).  Both networks must satisfy
    mlp_fusable(); follow with ClippedAdam.step()."""
    device, stream, ws, scalars, head, keep = _mlp_minibatch_args(
        policy, value, observations, actions, old_log_probs, advantages, returns, old_values,
        index, clip_ratio, vf_clip, value_coef, entropy_coef, scalars_out)
    _call("ppo_mlp_cat_grad_f32", device, stream, *head, scalars.data_ptr(), ws.data_ptr(),
          ws.numel(), stream)
    return _stats_dict(scalars)


def ppo_mlp_cat_step(
    policy: torch.nn.Module,
    value: torch.nn.Module,
    optimizer,
    observations: torch.Tensor,
    actions: torch.Tensor,
    old_log_probs: torch.Tensor,
    advantages: torch.Tensor,
    returns: torch.Tensor,
    old_values: Optional[torch.Tensor] = None,
    index: Optional[torch.Tensor] = None,
    clip_ratio: float = 0.2,
    vf_clip: Optional[float] = None,
    value_coef: float = 0.5,
    entropy_coef: float = 0.01,
    scalars_out: Optional[torch.Tensor] = None,
) -> tuple[LossStats, torch.Tensor]:
    """ppo_mlp_cat_grads followed by optimizer.step() (a ClippedAdam over
    list(policy.parameters()) + list(value.parameters()), in that order) as
    two launches (ppo_mlp_cat_step_f32: the gradient kernel, then the
    reduction with clip_grad_norm_ and Adam in one kernel; three launches
    when that kernel's grid does not fit on the device at once).
    Returns the loss scalars and the pre-clip gradient norm (0-d device
    tensors)."""
    from .optim import ClippedAdam

    expect = list(policy.parameters()) + list(value.parameters())
    if (not isinstance(optimizer, ClippedAdam) or len(optimizer.params) != len(expect)
            or any(a is not b for a, b in zip(optimizer.params, expect))):
        raise ValueError("optimizer must be a ClippedAdam over the policy's then the value "
                         "network's parameters")
    device, stream, ws, scalars, head, keep = _mlp_minibatch_args(
        policy, value, observations, actions, old_log_probs, advantages, returns, old_values,
        index, clip_ratio, vf_clip, value_coef, entropy_coef, scalars_out)
    hp, step = optimizer._fused_params()
    P = ctypes.c_void_p * len(expect)
    m = P(*[t.data_ptr() for t in optimizer.exp_avg])
    v = P(*[t.data_ptr() for t in optimizer.exp_avg_sq])
    norm = torch.empty((), dtype=torch.float32, device=device)
    _call("ppo_mlp_cat_step_f32", device, stream, *head, m, v, ctypes.byref(hp),
          scalars.data_ptr(), norm.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    optimizer._advance(step)
    return _stats_dict(scalars), norm


def mlp_act_categorical(
    policy: torch.nn.Module,
    value: torch.nn.Module,
    observations: torch.Tensor,
    uniforms: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
    observations_out: Optional[torch.Tensor] = None,
    actions_out: Optional[torch.Tensor] = None,
    log_probs_out: Optional[torch.Tensor] = None,
    values_out: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """PPOAgent.select_action (ppo.py:65-79) for N observations [N,D] in one
    launch: both MLPs' forward (networks as in ppo_mlp_cat_grads) and
    sample_categorical's inverse-CDF draw at `uniforms` [N] (torch.rand on
    the device from `generator` when not given).  Returns (actions int32 [N],
    log_probs [N], values [N]); the *_out tensors are written in place when
    given, and observations_out (e.g. a rollout buffer row) receives a copy
    of the observations."""
    if not mlp_fusable(policy, value):
        raise ValueError("policy/value are not MLPs the fused kernel supports (see mlp_fusable)")
    lp, act = mlp_structure(policy)
    lv, _ = mlp_structure(value)
    D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
    device = lp[0].weight.device
    _require(observations, "observations", (torch.float32,), device)
    if observations.dim() != 2 or observations.shape[1] != D:
        raise ValueError(f"observations must be [N,{D}], got {tuple(observations.shape)}")
    N = observations.shape[0]
    if uniforms is None:
        uniforms = torch.rand(N, device=device, generator=generator)
    _require(uniforms, "uniforms", (torch.float32,), device)
    if uniforms.shape != (N,):
        raise ValueError(f"uniforms must be [N]=[{N}], got {tuple(uniforms.shape)}")
    if observations_out is not None:
        _require(observations_out, "observations_out", (torch.float32,), device)
        if observations_out.numel() != N * D:
            raise ValueError("observations_out must hold N x D values")
    actions_out = _out(actions_out, "actions_out", (N,), torch.int32, device)
    log_probs_out = _out(log_probs_out, "log_probs_out", (N,), torch.float32, device)
    values_out = _out(values_out, "values_out", (N,), torch.float32, device)
    s_actor, s_critic = _lib.Mlp3(), _lib.Mlp3()
    for st, layers in ((s_actor, lp), (s_critic, lv)):
        for i, m in enumerate(layers):
            st.weight[i] = m.weight.data_ptr()
            st.bias[i] = m.bias.data_ptr()
    stream = _stream(device)
    _call("ppo_mlp_act_cat_f32", device, stream, ctypes.byref(s_actor), ctypes.byref(s_critic),
          D, H, A, _lib.PPO_ACT_TANH if act == "tanh" else _lib.PPO_ACT_RELU,
          observations.data_ptr(), N, uniforms.data_ptr(), _ptr(observations_out),
          actions_out.data_ptr(), log_probs_out.data_ptr(), values_out.data_ptr(), stream)
    return actions_out, log_probs_out, values_out


def mlp_forward_categorical(
    policy: torch.nn.Module,
    value: torch.nn.Module,
    observations: torch.Tensor,
    logits_out: Optional[torch.Tensor] = None,
    values_out: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """policy(observations) and value(observations).squeeze(-1) for
    observations [N,D] in one launch (ppo_mlp_forward_cat_f32; networks as in
    ppo_mlp_cat_grads).  Returns (logits [N,A], values [N]), written into
    logits_out / values_out when given.  Any of the three tensors may be
    pinned host memory, which the kernel reads and writes over the bus (the
    forward half of PPOAgent.select_action, ppo.py:65-79: observation in,
    logits and value out, one synchronisation and no copy launch); results in
    host memory are valid once the stream is synchronised."""
    if not mlp_fusable(policy, value):
        raise ValueError("policy/value are not MLPs the fused kernel supports (see mlp_fusable)")
    lp, act = mlp_structure(policy)
    lv, _ = mlp_structure(value)
    D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
    device = lp[0].weight.device

    def check(t, name, shape):
        # a device tensor on the networks' GPU, or pinned host memory
        if isinstance(t, torch.Tensor) and t.device.type == "cpu" and t.is_pinned():
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise TypeError(f"{name} must be contiguous fp32")
        else:
            _require(t, name, (torch.float32,), device)
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")

    if not isinstance(observations, torch.Tensor) or observations.dim() != 2:
        raise ValueError("observations must be a [N,D] tensor")
    N = observations.shape[0]
    check(observations, "observations", (N, D))
    if logits_out is None:
        logits_out = torch.empty((N, A), dtype=torch.float32, device=device)
    if values_out is None:
        values_out = torch.empty((N,), dtype=torch.float32, device=device)
    check(logits_out, "logits_out", (N, A))
    check(values_out, "values_out", (N,))
    s_actor, s_critic = _lib.Mlp3(), _lib.Mlp3()
    for st, layers in ((s_actor, lp), (s_critic, lv)):
        for i, m in enumerate(layers):
            st.weight[i] = m.weight.data_ptr()
            st.bias[i] = m.bias.data_ptr()
    stream = _stream(device)
    _call("ppo_mlp_forward_cat_f32", device, stream, ctypes.byref(s_actor),
          ctypes.byref(s_critic), D, H, A,
          _lib.PPO_ACT_TANH if act == "tanh" else _lib.PPO_ACT_RELU,
          observations.data_ptr(), N, logits_out.data_ptr(), values_out.data_ptr(), stream)
    return logits_out, values_out


def mlp_cartpole_rollout(
    policy: torch.nn.Module,
    value: torch.nn.Module,
    env,
    buffer,
    observations: torch.Tensor,
    action_uniforms: torch.Tensor,
    reset_uniforms: torch.Tensor,
) -> torch.Tensor:
    """A whole rollout of `buffer.T` steps of `env` (a CartPoleVec) in one
    launch (ppo_cartpole_rollout_f32): per step mlp_act_categorical at
    action_uniforms[t] ([T,N] rows, any row stride) and env.step_into with
    reset_uniforms[t] ([T,N,4] rows), filling buffer rows 0..T-1 (the caller
    sets buffer.step).  Starts from `observations` [N,4]; returns env.obs,
    which holds the observations after the last step.  The results equal the
    step-by-step path's on the same uniforms."""
    if not mlp_fusable(policy, value):
        raise ValueError("policy/value are not MLPs the fused kernel supports (see mlp_fusable)")
    lp, act = mlp_structure(policy)
    lv, _ = mlp_structure(value)
    D, H, A = lp[0].in_features, lp[0].out_features, lp[2].out_features
    if D != 4 or A != 2:
        raise ValueError(f"the CartPole rollout needs 4-H-H-2 / 4-H-H-1 networks, got D={D}, A={A}")
    device = env.device
    T, N = buffer.T, buffer.N
    if N != env.num_envs:
        raise ValueError(f"buffer has N={N}, the environment {env.num_envs}")
    if buffer.actions.dtype != torch.int32 or buffer.actions.dim() != 2:
        raise ValueError("the rollout buffer must hold categorical int32 actions")
    if tuple(buffer.observations.shape) != (T, N, 4) or buffer.observations.device != device:
        raise ValueError("the rollout buffer must hold [T,N,4] observations on the env's device")
    _require(observations, "observations", (torch.float32,), device)
    if tuple(observations.shape) != (N, 4):
        raise ValueError(f"observations must be [N,4]=[{N},4], got {tuple(observations.shape)}")
    if (action_uniforms.dtype != torch.float32 or action_uniforms.device != device
            or tuple(action_uniforms.shape) != (T, N) or action_uniforms.stride(1) != 1):
        raise ValueError("action_uniforms must be fp32 [T,N] rows of unit stride on the device")
    if (reset_uniforms.dtype != torch.float32 or reset_uniforms.device != device
            or tuple(reset_uniforms.shape) != (T, N, 4) or reset_uniforms.stride(2) != 1
            or reset_uniforms.stride(1) != 4):
        raise ValueError("reset_uniforms must be fp32 [T,N,4] with contiguous rows on the device")
    s_actor, s_critic = _lib.Mlp3(), _lib.Mlp3()
    for st, layers in ((s_actor, lp), (s_critic, lv)):
        for i, m in enumerate(layers):
            st.weight[i] = m.weight.data_ptr()
            st.bias[i] = m.bias.data_ptr()
    stream = _stream(device)
    _call("ppo_cartpole_rollout_f32", device, stream, ctypes.byref(s_actor),
          ctypes.byref(s_critic), H, _lib.PPO_ACT_TANH if act == "tanh" else _lib.PPO_ACT_RELU,
          N, T, env.max_steps, env.state.data_ptr(), env.steps.data_ptr(),
          observations.data_ptr(), env.obs.data_ptr(), action_uniforms.data_ptr(),
          action_uniforms.stride(0), reset_uniforms.data_ptr(), reset_uniforms.stride(0),
          buffer.observations.data_ptr(), buffer.actions.data_ptr(),
          buffer.log_probs.data_ptr(), buffer.values.data_ptr(), buffer.rewards.data_ptr(),
          buffer.dones.data_ptr(), env._ret.data_ptr(), env._done_sum.data_ptr(),
          env._done_count.data_ptr(), stream)
    return env.obs
