"""ctypes binding of libppo_amd.so, the C ABI declared in include/ppo_amd.h.

The library is built in-tree (ppo_amd/build.py or csrc/Makefile) and loaded
from this directory.  There is no fallback: if the library is missing or does
not load, every op raises.
"""

from __future__ import annotations

import ctypes
import os

LIB_NAME = "libppo_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

PPO_OK = 0
PPO_NUM_SCALARS = 6
SCALAR_NAMES = ("loss", "policy", "value", "entropy", "approx_kl", "clipfrac")


class LossParams(ctypes.Structure):
    """struct ppo_loss_params (include/ppo_amd.h)."""

    _fields_ = [
        ("clip_ratio", ctypes.c_double),
        ("vf_clip", ctypes.c_double),
        ("value_coef", ctypes.c_double),
        ("entropy_coef", ctypes.c_double),
    ]


class AdamParams(ctypes.Structure):
    """struct ppo_adam_params (include/ppo_amd.h)."""

    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("max_grad_norm", ctypes.c_double),
        ("step", ctypes.c_int64),
        ("step_counter", ctypes.c_void_p),
    ]


class Mlp3(ctypes.Structure):
    """struct ppo_mlp3_f32 (include/ppo_amd.h): the three nn.Linear layers of
    an MLP and their gradient buffers, as device pointers."""

    _fields_ = [
        ("weight", ctypes.c_void_p * 3),
        ("bias", ctypes.c_void_p * 3),
        ("weight_grad", ctypes.c_void_p * 3),
        ("bias_grad", ctypes.c_void_p * 3),
    ]


GAE_ROUTES = {0: "none", 1: "resident", 2: "strip", 3: "span", 4: "tiles"}

PPO_ACT_RELU = 0
PPO_ACT_TANH = 1
PPO_ERR_UNSUPPORTED = 4
PPO_ERR_WAIT_TIMEOUT = 5

GATHER_MAX_ARRAYS = 8
ADAM_MAX_TENSORS = 32

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f64 = ctypes.c_double
_sz = ctypes.c_size_t
_int = ctypes.c_int

# name -> (restype, argtypes); one entry per function in include/ppo_amd.h
SIGNATURES = {
    "ppo_amd_version": (_int, []),
    "ppo_amd_strerror": (ctypes.c_char_p, [_int]),
    "ppo_wait_status": (_int, [_vp]),
    "ppo_wait_status_async": (_int, [_vp, _vp]),
    "ppo_wait_reset": (_int, [_vp]),
    "ppo_set_wait_limit": (_int, [_i64]),
    "ppo_gae_workspace_bytes": (_sz, [_i64, _i64]),
    "ppo_gae_route": (_int, [_i64, _i64, _int, _int]),
    "ppo_gae_f32": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _i64, _f64, _f64, _vp, _vp, _vp, _sz, _vp],
    ),
    "ppo_gae_norm_f32": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _i64, _f64, _f64, _f64, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "ppo_adv_norm_workspace_bytes": (_sz, [_i64]),
    "ppo_adv_norm_f32": (_int, [_vp, _i64, _f64, _vp, _vp, _vp, _sz, _vp]),
    "ppo_loss_cat_workspace_bytes": (_sz, [_i64, _i32]),
    "ppo_loss_cat_f32": (
        _int,
        [_vp, _i64, _i32, _vp, _int, _vp, _vp, _vp, _vp, _vp,
         ctypes.POINTER(LossParams), _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "ppo_loss_cat_f32_noalloc": (
        _int,
        [_vp, _i64, _i32, _vp, _int, _vp, _vp, _vp, _vp, _vp,
         ctypes.POINTER(LossParams), _vp, _vp, _vp, _vp],
    ),
    "ppo_loss_gauss_workspace_bytes": (_sz, [_i64, _i32]),
    "ppo_loss_gauss_f32": (
        _int,
        [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
         ctypes.POINTER(LossParams), _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "ppo_gather_rows": (
        _int,
        [_vp, _i64, _i64, _i32,
         ctypes.POINTER(_vp), ctypes.POINTER(_i32), ctypes.POINTER(_vp), _vp],
    ),
    "ppo_copy_from_pinned": (_int, [_vp, _vp, _i64, _vp]),
    "ppo_cartpole_reset": (_int, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "ppo_cartpole_step": (
        _int, [_vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "ppo_cartpole_rollout_f32": (
        _int,
        [ctypes.POINTER(Mlp3), ctypes.POINTER(Mlp3), _i32, _i32, _i64, _i32, _i32, _vp, _vp, _vp,
         _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "ppo_mlp_act_cat_f32": (
        _int,
        [ctypes.POINTER(Mlp3), ctypes.POINTER(Mlp3), _i32, _i32, _i32, _i32, _vp, _i64, _vp, _vp,
         _vp, _vp, _vp, _vp],
    ),
    "ppo_mlp_forward_cat_f32": (
        _int,
        [ctypes.POINTER(Mlp3), ctypes.POINTER(Mlp3), _i32, _i32, _i32, _i32, _vp, _i64, _vp, _vp,
         _vp],
    ),
    "ppo_sample_cat_f32": (_int, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ppo_sample_gauss_f32": (_int, [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ppo_mlp_cat_grad_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32]),
    "ppo_mlp_cat_grad_f32": (
        _int,
        [ctypes.POINTER(Mlp3), ctypes.POINTER(Mlp3), _i32, _i32, _i32, _i32, _vp, _i64, _vp,
         _i64, _vp, _int, _vp, _vp, _vp, _vp, ctypes.POINTER(LossParams), _vp, _vp, _sz, _vp],
    ),
    "ppo_mlp_cat_step_f32": (
        _int,
        [ctypes.POINTER(Mlp3), ctypes.POINTER(Mlp3), _i32, _i32, _i32, _i32, _vp, _i64, _vp,
         _i64, _vp, _int, _vp, _vp, _vp, _vp, ctypes.POINTER(LossParams), ctypes.POINTER(_vp),
         ctypes.POINTER(_vp), ctypes.POINTER(AdamParams), _vp, _vp, _vp, _sz, _vp],
    ),
    "ppo_adam_clip_workspace_bytes": (_sz, [_i32, ctypes.POINTER(_i64)]),
    "ppo_adam_clip_f32": (
        _int,
        [_i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
         ctypes.POINTER(_vp), ctypes.POINTER(_i64), ctypes.POINTER(AdamParams), _vp, _vp, _sz,
         _vp],
    ),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libppo_amd.so once and attach the prototypes; raise if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built. Build it with `python -m ppo_amd.build` "
                "(or __graft_entry__.build()); ppo_amd has no CPU fallback."
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class PPOLibraryError(RuntimeError):
    """A non-zero return code from libppo_amd."""

    def __init__(self, fn: str, code: int) -> None:
        msg = load().ppo_amd_strerror(code).decode()
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


def check(fn: str, code: int) -> None:
    if code != PPO_OK:
        raise PPOLibraryError(fn, code)
