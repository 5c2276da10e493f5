"""bench.py contract checks that need no GPU: more than one GPU is refused
with a message, and the roofline traffic figure comes from the committed
rocprof summary of the attention launch."""

from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""


def test_traffic_comes_from_the_committed_profile():
    sys.path.insert(0, ROOT)
    import bench

    t = bench.profiled_traffic("headline")
    assert isinstance(t, int) and t > 0
    text = open(os.path.join(ROOT, "profiles", "attn_kernel_headline64k_traffic.txt")).read()
    assert f"attn_kernel traffic_bytes_per_step: {t}" in text
    # the calibrated traffic is at least the launch's algorithmic bytes (Q, K, staged V, O)
    assert t >= 32 * 65536 * 96 * 2 * 4
    assert bench.profiled_traffic("no_such_workload") is None
