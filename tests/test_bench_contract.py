"""bench.py's contract pieces that need no GPU: the roofline's traffic comes from the
committed decode profile under the kernel's own name, and more than one GPU is refused."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_decode_traffic_found_in_profile():
    t = bench.measured_traffic(bench.DECODE_PROFILE, bench.DECODE_KERNEL)
    assert t is not None and t > 1_000_000_000, t
    with open(os.path.join(ROOT, "profiles", bench.DECODE_PROFILE)) as f:
        assert bench.DECODE_KERNEL in f.read()  # the summary names the kernel it measured


def test_more_than_one_gpu_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
