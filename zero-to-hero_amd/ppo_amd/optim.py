"""clip_grad_norm_ + Adam as one fused GPU step (rl/deep/agents/ppo.py:170-171).

`ClippedAdam` holds the same state as torch.optim.Adam (exp_avg, exp_avg_sq
and a step count per parameter) and replaces the pair

    nn.utils.clip_grad_norm_(params, max_grad_norm)
    optimizer.step()

with two kernel launches (ppo_adam_clip_f32) whatever the number of tensors,
following torch's multi-tensor Adam operation by operation in fp32.

With `capturable=True` the step count lives in a device int64 counter that the
first kernel increments and the second turns into the bias corrections, so a
step() recorded in a CUDA/HIP graph advances the count on every replay (the
role of torch.optim.Adam(capturable=True)).
"""

from __future__ import annotations

import ctypes
from typing import Iterable

import torch

from . import _lib
from .ops import _WORKSPACES, _call, _stream


class ClippedAdam:
    """Adam (no weight decay, no amsgrad) on fp32 CUDA parameters whose
    gradients are first clipped to a global 2-norm of `max_grad_norm`
    (<= 0 disables clipping).  step() returns the pre-clip total norm as a
    0-d device tensor, as clip_grad_norm_ does."""

    def __init__(
        self,
        params: Iterable[torch.Tensor],
        lr: float = 3e-4,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        max_grad_norm: float = 0.5,
        capturable: bool = False,
    ) -> None:
        self.params = list(params)
        if not self.params:
            raise ValueError("ClippedAdam got an empty parameter list")
        if len(self.params) > _lib.ADAM_MAX_TENSORS:
            raise ValueError(f"at most {_lib.ADAM_MAX_TENSORS} tensors, got {len(self.params)}")
        device = self.params[0].device
        for k, p in enumerate(self.params):
            if p.device.type != "cuda" or p.device != device:
                raise RuntimeError(f"parameter {k} is on {p.device}; ClippedAdam runs on one GPU")
            if p.dtype != torch.float32 or not p.is_contiguous():
                raise TypeError(f"parameter {k} must be contiguous fp32")
        if not lr >= 0.0 or not eps >= 0.0:
            raise ValueError("lr and eps must be >= 0")
        self.device = device
        self.lr, self.betas, self.eps, self.max_grad_norm = lr, betas, eps, max_grad_norm
        self.exp_avg = [torch.zeros_like(p) for p in self.params]
        self.exp_avg_sq = [torch.zeros_like(p) for p in self.params]
        self.steps = [0] * len(self.params)
        self.capturable = capturable
        # device step counter (capturable mode): one count shared by all tensors
        self.step_t = (torch.zeros((), dtype=torch.int64, device=device)
                       if capturable else None)

    def step_count(self) -> int:
        """The number of steps taken (reads the device counter in capturable
        mode, which synchronises)."""
        if self.capturable:
            return int(self.step_t.item())
        return max(self.steps)

    # True when the parameters' gradient buffers must keep their storage
    # (captured graphs and the fused MLP step write into them): zero_grad then
    # zeroes them in place whatever set_to_none says.
    keep_grads = False

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if p.grad is not None:
                if set_to_none and not self.keep_grads:
                    p.grad = None
                else:
                    p.grad.zero_()

    def state_dict(self) -> dict:
        """The state in torch.optim.Adam's layout (per parameter index:
        step, exp_avg, exp_avg_sq; one param group), so that it can be saved,
        and loaded into either optimizer."""
        if self.capturable:
            steps = [self.step_t.detach().to(torch.float32).cpu()] * len(self.params)
        else:
            steps = [torch.tensor(float(k)) for k in self.steps]
        state = {i: {"step": steps[i].clone(), "exp_avg": self.exp_avg[i].detach().clone(),
                     "exp_avg_sq": self.exp_avg_sq[i].detach().clone()}
                 for i in range(len(self.params))}
        group = {"lr": self.lr, "betas": tuple(self.betas), "eps": self.eps,
                 "weight_decay": 0.0, "amsgrad": False, "max_grad_norm": self.max_grad_norm,
                 "params": list(range(len(self.params)))}
        return {"state": state, "param_groups": [group]}

    @torch.no_grad()
    def load_state_dict(self, state_dict: dict) -> None:
        """Loads a state_dict() of this class or of torch.optim.Adam over the
        same parameters (one group, no weight decay, no amsgrad), copying the
        moments into the existing buffers (their storage stays, as captured
        graphs need).  Parameters absent from the state start at step 0."""
        groups = state_dict["param_groups"]
        if len(groups) != 1 or len(groups[0]["params"]) != len(self.params):
            raise ValueError("expected one parameter group over the same parameters")
        g = groups[0]
        if g.get("weight_decay", 0.0) or g.get("amsgrad", False):
            raise ValueError("ClippedAdam has no weight decay and no amsgrad")
        self.lr, self.betas, self.eps = g["lr"], tuple(g["betas"]), g["eps"]
        self.max_grad_norm = g.get("max_grad_norm", self.max_grad_norm)
        steps = []
        for i, key in enumerate(g["params"]):
            st = state_dict["state"].get(key)
            if st is None:
                self.exp_avg[i].zero_()
                self.exp_avg_sq[i].zero_()
                steps.append(0)
                continue
            self.exp_avg[i].copy_(st["exp_avg"])
            self.exp_avg_sq[i].copy_(st["exp_avg_sq"])
            steps.append(int(float(st["step"])))
        if self.capturable:
            if len(set(steps)) != 1:
                raise ValueError("capturable mode keeps one step count for all parameters")
            self.step_t.fill_(steps[0])
        else:
            self.steps = steps

    def _fused_params(self) -> tuple:
        """Adam parameters for a fused step of all tensors together (the
        gradients written by the same launch sequence) and the step number
        it makes."""
        if not self.capturable and len(set(self.steps)) != 1:
            raise RuntimeError("a fused step needs every parameter at the same step count")
        step = self.steps[0] + 1
        hp = _lib.AdamParams(float(self.lr), float(self.betas[0]), float(self.betas[1]),
                             float(self.eps), float(self.max_grad_norm), int(step),
                             self.step_t.data_ptr() if self.capturable else None)
        return hp, step

    def _advance(self, step: int) -> None:
        if not self.capturable:
            self.steps = [step] * len(self.params)

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        # as torch: parameters without a gradient are skipped (and keep their step)
        live = [k for k, p in enumerate(self.params) if p.grad is not None]
        if not live:
            return torch.zeros((), dtype=torch.float32, device=self.device)
        # written by the kernel (no fill launch)
        norm = torch.empty((), dtype=torch.float32, device=self.device)
        if self.capturable and len(live) != len(self.params):
            raise RuntimeError("ClippedAdam(capturable=True) steps all parameters together; "
                               "every parameter needs a gradient")
        for k in live:
            g = self.params[k].grad
            if g.dtype != torch.float32 or not g.is_contiguous():
                raise TypeError(f"gradient of parameter {k} must be contiguous fp32")
        # one launch pair per group of tensors at the same step count (one group
        # in steady state); the clip norm spans all live gradients only when
        # they form one group, so mixed counts are stepped without clipping
        groups: dict[int, list[int]] = {}
        for k in live:
            groups.setdefault(self.steps[k] + 1, []).append(k)
        if len(groups) > 1 and self.max_grad_norm > 0:
            raise RuntimeError("ClippedAdam: parameters at different step counts cannot share "
                               "one clip norm; step them together from the start")
        stream = _stream(self.device)
        lib = _lib.load()
        for step, ks in groups.items():
            nt = len(ks)
            P = ctypes.c_void_p * nt
            numel = (ctypes.c_int64 * nt)(*[self.params[k].numel() for k in ks])
            hp = _lib.AdamParams(float(self.lr), float(self.betas[0]), float(self.betas[1]),
                                 float(self.eps), float(self.max_grad_norm), int(step),
                                 self.step_t.data_ptr() if self.capturable else None)
            nbytes = lib.ppo_adam_clip_workspace_bytes(nt, numel)
            ws = _WORKSPACES.get(self.device, stream, nbytes)
            _call(
                "ppo_adam_clip_f32", self.device, stream, nt,
                P(*[self.params[k].data_ptr() for k in ks]),
                P(*[self.params[k].grad.data_ptr() for k in ks]),
                P(*[self.exp_avg[k].data_ptr() for k in ks]),
                P(*[self.exp_avg_sq[k].data_ptr() for k in ks]),
                numel, ctypes.byref(hp), norm.data_ptr(), ws.data_ptr(), ws.numel(), stream,
            )
            if not self.capturable:
                for k in ks:
                    self.steps[k] = step
        return norm
