"""The C-ABI library loads and exports every function include/ppo_amd.h
declares, with the prototypes the ctypes binding attaches; host-side argument
checks return their error codes before any device work.  CPU only: no
function here launches a kernel."""

import ctypes
import os
import re

import pytest

from ppo_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ppo_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ppo_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_functions():
    names = declared_functions()
    assert "ppo_gae_f32" in names and "ppo_loss_cat_f32" in names
    assert len(names) == 31


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"no ctypes prototype for {name}"
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_nm_shows_c_linkage():
    syms = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    for name in declared_functions():
        assert re.search(rf"\bT {name}$", syms, flags=re.M), name
    # and nothing else: the library is built with hidden visibility
    exported = set(re.findall(r"\bT (\S+)$", syms, flags=re.M))
    assert exported == set(declared_functions()), sorted(exported ^ set(declared_functions()))


def test_version_and_strerror():
    lib = _lib.load()
    assert lib.ppo_amd_version() == 200
    assert lib.ppo_amd_strerror(0) == b"ok"
    assert b"workspace" in lib.ppo_amd_strerror(2)
    assert lib.ppo_amd_strerror(12345) != b""


def test_workspace_queries():
    lib = _lib.load()
    assert lib.ppo_gae_workspace_bytes(0, 0) == 256
    small = lib.ppo_gae_workspace_bytes(128, 8)
    big = lib.ppo_gae_workspace_bytes(2048, 4096)
    assert 256 < small < big
    # summary (16 B) + carry (8 B) + five fp32 tile sums (20 B) per env per
    # tile, tiles of >= 16 steps
    assert big < 2048 * 4096 * 44 / 16 + (1 << 20)
    assert lib.ppo_adv_norm_workspace_bytes(1 << 23) > 256
    assert lib.ppo_loss_cat_workspace_bytes(1 << 20, 18) > 256
    assert lib.ppo_loss_gauss_workspace_bytes(1 << 21, 6) > 256


def test_host_side_errors_before_launch():
    lib = _lib.load()
    # negative sizes
    assert lib.ppo_gae_f32(None, None, None, None, -1, 4, 0.99, 0.95, None, None, None, 0,
                           None) == 1
    # zero-size work is a no-op success
    assert lib.ppo_gae_f32(None, None, None, None, 0, 4, 0.99, 0.95, None, None, None, 0,
                           None) == 0
    # null inputs
    assert lib.ppo_gae_f32(None, None, None, None, 4, 4, 0.99, 0.95, None, None, None, 0,
                           None) == 1
    # workspace too small (non-null dummy pointers never dereferenced)
    p = ctypes.c_void_p(256)
    assert lib.ppo_gae_f32(p, p, p, None, 4096, 4096, 0.99, 0.95, p, p, p, 16, None) == 2
    assert lib.ppo_adv_norm_f32(None, -3, 1e-8, None, None, None, 0, None) == 1
    params = _lib.LossParams(0.2, 0.0, 0.5, 0.01)
    assert lib.ppo_loss_cat_f32(None, 0, 4, None, 0, None, None, None, None, None,
                                ctypes.byref(params), None, None, None, None, 0, None) == 1
    assert lib.ppo_loss_gauss_f32(p, p, 10, 25, p, p, p, p, p, None, ctypes.byref(params),
                                  p, p, p, p, p, 1 << 20, None) == 3
    # sampling: A <= 0 / null outputs / D above the limit; N == 0 is a no-op
    assert lib.ppo_sample_cat_f32(p, 4, 0, p, p, p, None, None, None) == 1
    assert lib.ppo_sample_cat_f32(p, 4, 3, p, None, p, None, None, None) == 1
    assert lib.ppo_sample_cat_f32(None, 0, 3, None, None, None, None, None, None) == 0
    assert lib.ppo_sample_gauss_f32(p, p, 4, 25, p, p, p, None, None, None) == 3
    # gather: 8 arrays of 2^29 - 1 words per row (~2^32 words) exceed the kernel's
    # 2^30-word row table; rows that are not whole words are refused
    ptrs = (ctypes.c_void_p * 8)(*([256] * 8))
    wide = (ctypes.c_int32 * 8)(*([2**31 - 4] * 8))
    assert lib.ppo_gather_rows(p, 4, 4, 8, ptrs, wide, ptrs, None) == 3
    odd = (ctypes.c_int32 * 8)(*([6] * 8))
    assert lib.ppo_gather_rows(p, 4, 4, 8, ptrs, odd, ptrs, None) == 1
    # Adam: a negative tensor size is an argument error, checked before the workspace
    numel = (ctypes.c_int64 * 1)(-8)
    hp = _lib.AdamParams(1e-3, 0.9, 0.999, 1e-8, 0.5, 1, None)
    assert lib.ppo_adam_clip_f32(1, ptrs, ptrs, ptrs, ptrs, numel, ctypes.byref(hp), None,
                                 None, 0, None) == 1


def test_error_mapping():
    with pytest.raises(_lib.PPOLibraryError, match="workspace"):
        _lib.check("ppo_gae_f32", 2)
