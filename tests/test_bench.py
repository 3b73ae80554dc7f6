"""bench.py's host side, without a GPU: the multi-GPU refusal and the HBM
traffic figure it reads from the committed loss profile (which must agree
with the loss's algorithmic bytes: a mis-scaled PMC calibration shows up here
as a traffic far from 172 B/sample)."""

import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr + p.stdout


def test_profile_traffic_matches_algorithmic_bytes():
    traffic = bench.read_traffic("loss_cat_north_star")
    alg = bench.LOSS_CAT_BYTES * bench.T_STEPS * bench.N_ENVS
    assert traffic is not None
    assert 0.99 * alg <= traffic <= 1.05 * alg, (traffic, alg)


def _bytes_per_element(name):
    import re

    text = open(os.path.join(ROOT, "profiles", f"{name}.md")).read()
    m = re.search(r"Total HBM bytes per call: \d+ \(([0-9.]+) B/element", text)
    assert m, name
    return float(m.group(1))


def test_gae_profiles_traffic_near_algorithmic_bytes():
    # 21 and 17 algorithmic bytes per element; the resident pass re-reads
    # only each segment's following value row and its slots
    assert 21.0 <= _bytes_per_element("gae_norm_config2") <= 23.0
    assert 17.0 <= _bytes_per_element("gae_resident_config3") <= 20.0
